// The launch manifest a libhwk code object carries: for each kernel, the workgroup size and how the
// grid follows from the kernel's arguments, so that a caller never passes grid or block sizes (the
// reference's Run has no geometry parameters: the NPU's comes from the xclbin, internal/backend/amd/
// device.go:304-338). It is the constant array `hwk_co_manifest` (hwk_co_manifest_count entries) in
// the code object's read-only data, which the runtime reads from the ELF image itself.
#pragma once

#include <stdint.h>

#define HWK_CO_MANIFEST_SYMBOL "hwk_co_manifest"
#define HWK_CO_MANIFEST_COUNT_SYMBOL "hwk_co_manifest_count"
#define HWK_CO_FIXED_GRID 0xffffffffu

struct hwk_co_geometry {
  char kernel[64];       // the kernel's symbol name
  uint32_t block;        // threads a workgroup (x)
  uint32_t grid_arg;     // index of the 4-byte argument sizing grid.x, or HWK_CO_FIXED_GRID
  uint32_t grid_div;     // grid.x = ceil(argument / grid_div) (a fixed grid: grid.x = grid_div)
  uint32_t grid_per_cu;  // grid.x at most grid_per_cu * the device's CUs (0: no cap)
  uint32_t lds_bytes;    // dynamic LDS a workgroup
  uint32_t nullable;     // bit i: buffer argument i may be the null address (hwk_run_set_null)
  uint32_t reserved[2];
};
