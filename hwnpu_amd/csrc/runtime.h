// The device and buffer objects of libhwk's runtime calls (runtime.hip), shared with the code-object
// calls (codeobj.hip).
#pragma once

#include "hwk_common.h"

struct hwk_device {
  int index;
  hipDeviceProp_t prop;
};

struct hwk_buf {
  hwk_device *dev;
  size_t size;
  int kind;
  void *host;  // pinned mirror (HWK_BUF_MIRRORED), else null
  void *ptr;   // device allocation
};
