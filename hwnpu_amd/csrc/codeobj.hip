// libhwk's code-object calls: a gfx950 code object loaded as a program whose kernels are listed
// from the object's own metadata, and runs that take arguments by index with size checks and
// launch with the geometry the object's manifest gives (reference KernelDevice.LoadProgram,
// Program.Kernels/NewRun, Run.SetArg/SetBuffer/Submit, Fence; internal/backend/backend.go:27-46,
// internal/types/kernel.go:22-36, internal/backend/amd/device.go:304-420, kernel.go:109-254).
//
// The kernel list comes from the AMDGPU metadata note of the ELF (NT_AMDGPU_METADATA, a msgpack
// map): each kernel's name, its explicit arguments (offset, size, buffer or value, name) and the
// size of its argument buffer. The launch geometry comes from the `hwk_co_manifest` array in the
// object's read-only data (co_manifest.h). Both are read from the image bytes, so a module loaded
// without a device (for inspection) lists its kernels too. A clang offload bundle is accepted and
// its gfx950 entry used.
#include <algorithm>
#include <chrono>
#include <string>
#include <thread>
#include <utility>
#include <vector>

#include "co_manifest.h"
#include "runtime.h"

namespace {

// ---- msgpack (the subset the AMDGPU metadata uses) ----

struct Mp {
  enum Kind { NIL, BOOL, INT, FLT, STR, ARR, MAP } k = NIL;
  int64_t i = 0;
  double f = 0;
  std::string s;
  std::vector<Mp> a;
  std::vector<std::pair<std::string, Mp>> m;
  const Mp *get(const char *key) const {
    if (k != MAP) return nullptr;
    for (const auto &kv : m)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

struct MpReader {
  const uint8_t *p, *end;
  bool have(size_t n) const { return (size_t)(end - p) >= n; }
  uint64_t be(int n) {
    uint64_t v = 0;
    for (int j = 0; j < n; j++) v = v << 8 | p[j];
    p += n;
    return v;
  }
  bool bytes(size_t n, std::string &out) {
    if (!have(n)) return false;
    out.assign((const char *)p, n);
    p += n;
    return true;
  }
  bool read(Mp &o, int depth) {
    if (depth > 32 || !have(1)) return false;
    const uint8_t b = *p++;
    auto len = [&](int n, uint64_t &v) {
      if (!have(n)) return false;
      v = be(n);
      return true;
    };
    uint64_t n = 0;
    if (b <= 0x7f) { o.k = Mp::INT; o.i = b; return true; }
    if (b >= 0xe0) { o.k = Mp::INT; o.i = (int8_t)b; return true; }
    if ((b & 0xf0) == 0x80) return map(o, b & 0x0f, depth);
    if ((b & 0xf0) == 0x90) return arr(o, b & 0x0f, depth);
    if ((b & 0xe0) == 0xa0) { o.k = Mp::STR; return bytes(b & 0x1f, o.s); }
    switch (b) {
      case 0xc0: o.k = Mp::NIL; return true;
      case 0xc2: o.k = Mp::BOOL; o.i = 0; return true;
      case 0xc3: o.k = Mp::BOOL; o.i = 1; return true;
      case 0xc4: case 0xc5: case 0xc6:
        if (!len(1 << (b - 0xc4), n)) return false;
        o.k = Mp::STR;
        return bytes(n, o.s);
      case 0xca: {
        if (!have(4)) return false;
        const uint32_t u = (uint32_t)be(4);
        float f;
        memcpy(&f, &u, 4);
        o.k = Mp::FLT; o.f = f;
        return true;
      }
      case 0xcb: {
        if (!have(8)) return false;
        const uint64_t u = be(8);
        memcpy(&o.f, &u, 8);
        o.k = Mp::FLT;
        return true;
      }
      case 0xcc: case 0xcd: case 0xce: case 0xcf:
        if (!len(1 << (b - 0xcc), n)) return false;
        o.k = Mp::INT; o.i = (int64_t)n;
        return true;
      case 0xd0: case 0xd1: case 0xd2: case 0xd3: {
        const int w = 1 << (b - 0xd0);
        if (!len(w, n)) return false;
        o.k = Mp::INT;
        o.i = w == 8 ? (int64_t)n : (int64_t)(n << (64 - 8 * w)) >> (64 - 8 * w);
        return true;
      }
      case 0xd9: case 0xda: case 0xdb:
        if (!len(1 << (b - 0xd9), n)) return false;
        o.k = Mp::STR;
        return bytes(n, o.s);
      case 0xdc: case 0xdd:
        if (!len(b == 0xdc ? 2 : 4, n)) return false;
        return arr(o, n, depth);
      case 0xde: case 0xdf:
        if (!len(b == 0xde ? 2 : 4, n)) return false;
        return map(o, n, depth);
      default: return false;  // ext types: not in the metadata
    }
  }
  bool arr(Mp &o, uint64_t n, int depth) {
    if (n > (uint64_t)(end - p)) return false;
    o.k = Mp::ARR;
    o.a.resize(n);
    for (auto &e : o.a)
      if (!read(e, depth + 1)) return false;
    return true;
  }
  bool map(Mp &o, uint64_t n, int depth) {
    if (n > (uint64_t)(end - p)) return false;
    o.k = Mp::MAP;
    o.m.resize(n);
    for (auto &kv : o.m) {
      Mp key;
      if (!read(key, depth + 1) || key.k != Mp::STR) return false;
      kv.first = key.s;
      if (!read(kv.second, depth + 1)) return false;
    }
    return true;
  }
};

// ---- ELF64 (little endian) ----

template <typename T>
bool rd(const uint8_t *img, size_t n, size_t off, T &v) {
  if (off > n || n - off < sizeof(T)) return false;
  memcpy(&v, img + off, sizeof(T));
  return true;
}

struct Section {
  uint32_t name, type;
  uint64_t addr, off, size, entsize;
  uint32_t link;
};

bool elf_sections(const uint8_t *img, size_t n, std::vector<Section> &out) {
  if (n < 64 || memcmp(img, "\x7f" "ELF", 4) != 0 || img[4] != 2 || img[5] != 1) return false;
  uint64_t shoff;
  uint16_t shentsize, shnum;
  if (!rd(img, n, 0x28, shoff) || !rd(img, n, 0x3a, shentsize) || !rd(img, n, 0x3c, shnum)) return false;
  if (shentsize < 64) return false;
  for (uint32_t i = 0; i < shnum; i++) {
    const size_t b = shoff + (size_t)i * shentsize;
    Section s;
    if (!rd(img, n, b, s.name) || !rd(img, n, b + 4, s.type) || !rd(img, n, b + 16, s.addr) ||
        !rd(img, n, b + 24, s.off) || !rd(img, n, b + 32, s.size) || !rd(img, n, b + 40, s.link) ||
        !rd(img, n, b + 56, s.entsize))
      return false;
    out.push_back(s);
  }
  return true;
}

// The msgpack bytes of the NT_AMDGPU_METADATA note (owner "AMDGPU", type 32).
bool elf_metadata(const uint8_t *img, size_t n, const std::vector<Section> &secs, const uint8_t **md, size_t *mdn) {
  for (const Section &s : secs) {
    if (s.type != 7 /* SHT_NOTE */ || s.off > n || s.size > n - s.off) continue;
    size_t p = s.off;
    const size_t end = s.off + s.size;
    while (p + 12 <= end) {
      uint32_t namesz, descsz, type;
      rd(img, n, p, namesz);
      rd(img, n, p + 4, descsz);
      rd(img, n, p + 8, type);
      const size_t name_off = p + 12, desc_off = name_off + ((namesz + 3) & ~3u);
      if (desc_off > end || descsz > end - desc_off) return false;
      if (type == 32 && namesz >= 6 && memcmp(img + name_off, "AMDGPU", 6) == 0) {
        *md = img + desc_off;
        *mdn = descsz;
        return true;
      }
      p = desc_off + ((descsz + 3) & ~3u);
    }
  }
  return false;
}

// The bytes of a symbol's initial data (a defined object in an allocated section with contents).
bool elf_symbol(const uint8_t *img, size_t n, const std::vector<Section> &secs, const char *want,
                const uint8_t **data, size_t *size) {
  for (const Section &s : secs) {
    if (s.type != 2 /* SHT_SYMTAB */ && s.type != 11 /* SHT_DYNSYM */) continue;
    if (s.link >= secs.size() || s.entsize < 24 || s.off > n || s.size > n - s.off) continue;
    const Section &str = secs[s.link];
    for (uint64_t k = 0; k < s.size / s.entsize; k++) {
      const size_t b = s.off + k * s.entsize;
      uint32_t nm;
      uint16_t shndx;
      uint64_t value, sz;
      if (!rd(img, n, b, nm) || !rd(img, n, b + 6, shndx) || !rd(img, n, b + 8, value) || !rd(img, n, b + 16, sz))
        return false;
      if (nm >= str.size || str.off + nm >= n) continue;
      const char *name = (const char *)img + str.off + nm;
      const size_t maxlen = n - (str.off + nm);
      if (strnlen(name, maxlen) == maxlen || strcmp(name, want) != 0) continue;
      if (shndx == 0 || shndx >= secs.size()) continue;
      const Section &d = secs[shndx];
      if (d.type == 8 /* SHT_NOBITS */ || value < d.addr || value - d.addr > d.size || sz > d.size - (value - d.addr))
        return false;
      const uint64_t off = d.off + (value - d.addr);
      if (off > n || sz > n - off) return false;
      *data = img + off;
      *size = sz;
      return true;
    }
  }
  return false;
}

// The gfx950 ELF inside a clang offload bundle, or the image itself.
bool unbundle(const uint8_t *img, size_t n, const uint8_t **elf, size_t *elfn) {
  static const char kMagic[] = "__CLANG_OFFLOAD_BUNDLE__";
  if (n < 24 || memcmp(img, kMagic, 24) != 0) {
    *elf = img;
    *elfn = n;
    return true;
  }
  uint64_t count;
  if (!rd(img, n, 24, count)) return false;
  size_t p = 32;
  for (uint64_t i = 0; i < count; i++) {
    uint64_t off, size, tlen;
    if (!rd(img, n, p, off) || !rd(img, n, p + 8, size) || !rd(img, n, p + 16, tlen)) return false;
    p += 24;
    if (tlen > n || p > n - tlen) return false;
    const std::string triple((const char *)img + p, tlen);
    p += tlen;
    if (triple.find("amdgcn") != std::string::npos && triple.find("gfx950") != std::string::npos) {
      if (off > n || size > n - off) return false;
      *elf = img + off;
      *elfn = size;
      return true;
    }
  }
  return false;
}

// A HIP kernel's explicit arguments fit in 4 KiB.
constexpr uint32_t kMaxKernargBytes = 4096;

struct KArg {
  uint32_t index, offset, size;
  bool buffer;
  bool nullable = false;  // the manifest lets the caller pass the null address
  std::string name;
};

struct Kernel {
  std::string name;
  std::vector<KArg> args;  // explicit arguments, in signature order
  uint32_t kernarg_bytes = 0, max_block = 0, lds_static = 0;
  bool has_geom = false;
  hwk_co_geometry geom{};
  hipFunction_t fn = nullptr;
};

const char *type_of(const KArg &a) {
  if (a.buffer) return "void *";
  switch (a.size) {
    case 1: return "uint8_t";
    case 2: return "uint16_t";
    case 4: return "uint32_t";
    case 8: return "uint64_t";
    default: return "bytes";
  }
}

// Lists the kernels of a code object image (no device needed).
char *parse(const void *image, size_t n, std::vector<Kernel> &out) {
  const uint8_t *elf;
  size_t elfn;
  HWK_CHECK(unbundle((const uint8_t *)image, n, &elf, &elfn), "hwk_module_load: an offload bundle without a gfx950 entry");
  std::vector<Section> secs;
  HWK_CHECK(elf_sections(elf, elfn, secs), "hwk_module_load: not a 64-bit little-endian ELF code object");
  const uint8_t *md;
  size_t mdn;
  HWK_CHECK(elf_metadata(elf, elfn, secs, &md, &mdn), "hwk_module_load: no AMDGPU metadata note");
  Mp root;
  MpReader rdr{md, md + mdn};
  HWK_CHECK(rdr.read(root, 0) && root.k == Mp::MAP, "hwk_module_load: malformed AMDGPU metadata");
  const Mp *target = root.get("amdhsa.target");
  HWK_CHECK(target && target->k == Mp::STR && target->s.find("gfx950") != std::string::npos,
            "hwk_module_load: code object for %s, not gfx950", target && target->k == Mp::STR ? target->s.c_str() : "?");
  const Mp *kernels = root.get("amdhsa.kernels");
  HWK_CHECK(kernels && kernels->k == Mp::ARR, "hwk_module_load: no amdhsa.kernels in the metadata");
  for (const Mp &k : kernels->a) {
    const Mp *name = k.get(".name");
    HWK_CHECK(name && name->k == Mp::STR, "hwk_module_load: a kernel without a name");
    Kernel kk;
    kk.name = name->s;
    if (const Mp *v = k.get(".max_flat_workgroup_size")) kk.max_block = (uint32_t)v->i;
    if (const Mp *v = k.get(".group_segment_fixed_size")) kk.lds_static = (uint32_t)v->i;
    if (const Mp *args = k.get(".args"); args && args->k == Mp::ARR) {
      uint32_t idx = 0;
      for (const Mp &a : args->a) {
        const Mp *kind = a.get(".value_kind"), *off = a.get(".offset"), *size = a.get(".size");
        HWK_CHECK(kind && kind->k == Mp::STR && off && size, "hwk_module_load: kernel %s: malformed argument",
                  kk.name.c_str());
        if (kind->s.rfind("hidden_", 0) == 0) continue;  // filled by the runtime
        // offsets and sizes are checked in 64 bits against the explicit-argument limit before
        // they size the host's argument buffer
        HWK_CHECK(off->k == Mp::INT && size->k == Mp::INT && off->i >= 0 && size->i >= 1 &&
                      (uint64_t)off->i + (uint64_t)size->i <= kMaxKernargBytes,
                  "hwk_module_load: kernel %s: argument at offset %lld of %lld bytes (at most %u in all)",
                  kk.name.c_str(), (long long)off->i, (long long)size->i, kMaxKernargBytes);
        KArg ka;
        ka.index = idx++;
        ka.offset = (uint32_t)off->i;
        ka.size = (uint32_t)size->i;
        ka.buffer = kind->s == "global_buffer" || kind->s == "dynamic_shared_pointer";
        const Mp *an = a.get(".name");
        ka.name = an && an->k == Mp::STR ? an->s : "arg" + std::to_string(ka.index);
        kk.kernarg_bytes = std::max(kk.kernarg_bytes, ka.offset + ka.size);
        kk.args.push_back(ka);
      }
    }
    out.push_back(kk);
  }
  // the manifest (optional: without it, kernels are listed but cannot run)
  const uint8_t *cnt_p, *man_p;
  size_t cnt_n, man_n;
  if (elf_symbol(elf, elfn, secs, HWK_CO_MANIFEST_COUNT_SYMBOL, &cnt_p, &cnt_n) && cnt_n == 4 &&
      elf_symbol(elf, elfn, secs, HWK_CO_MANIFEST_SYMBOL, &man_p, &man_n)) {
    uint32_t cnt;
    memcpy(&cnt, cnt_p, 4);
    HWK_CHECK((uint64_t)cnt * sizeof(hwk_co_geometry) <= man_n, "hwk_module_load: manifest of %u entries in %zu bytes",
              cnt, man_n);
    for (uint32_t i = 0; i < cnt; i++) {
      hwk_co_geometry g;
      memcpy(&g, man_p + (size_t)i * sizeof g, sizeof g);
      g.kernel[sizeof g.kernel - 1] = 0;
      for (Kernel &kk : out)
        if (kk.name == g.kernel) {
          HWK_CHECK(g.block >= 1 && g.block <= 1024 && (!kk.max_block || g.block <= kk.max_block),
                    "hwk_module_load: manifest block %u for %s (at most %u)", g.block, g.kernel, kk.max_block);
          HWK_CHECK(g.grid_div >= 1, "hwk_module_load: manifest grid_div 0 for %s", g.kernel);
          if (g.grid_arg != HWK_CO_FIXED_GRID)
            HWK_CHECK(g.grid_arg < kk.args.size() && kk.args[g.grid_arg].size == 4 && !kk.args[g.grid_arg].buffer,
                      "hwk_module_load: manifest grid argument %u of %s is not a 4-byte value", g.grid_arg, g.kernel);
          for (uint32_t i = 0; i < 32; i++) {
            if (!(g.nullable >> i & 1)) continue;
            HWK_CHECK(i < kk.args.size() && kk.args[i].buffer,
                      "hwk_module_load: manifest marks argument %u of %s nullable, which is not a buffer", i, g.kernel);
            kk.args[i].nullable = true;
          }
          kk.geom = g;
          kk.has_geom = true;
        }
    }
  }
  return nullptr;
}

}  // namespace

struct hwk_module {
  hwk_device *dev = nullptr;  // null: loaded for inspection only
  hipModule_t mod = nullptr;
  std::vector<Kernel> kernels;
};

struct hwk_run {
  hwk_module *m;
  const Kernel *k;
  std::vector<uint8_t> args;  // the explicit argument buffer; unset value arguments stay zero
  std::vector<uint8_t> set;   // per argument: set since the run was made (buffers must be)
  char *first_err = nullptr;
  hipEvent_t done = nullptr;
  bool submitted = false;
};

namespace {

char *record(hwk_run *r, char *err) {
  if (err && !r->first_err) {
    r->first_err = (char *)malloc(strlen(err) + 1);
    if (r->first_err) strcpy(r->first_err, err);
  }
  return err;
}

const KArg *arg_of(hwk_run *r, uint32_t i) { return i < r->k->args.size() ? &r->k->args[i] : nullptr; }

}  // namespace

extern "C" {

HWK_API char *hwk_module_load(hwk_device *d, const void *image, size_t n, hwk_module **out) {
  HWK_CHECK(image && out && n > 0, "hwk_module_load: null argument");
  hwk_module *m = new hwk_module();
  if (char *err = parse(image, n, m->kernels)) {
    delete m;
    return err;
  }
  m->dev = d;
  if (d) {
    hipError_t e = hipSetDevice(d->index);
    if (e == hipSuccess) e = hipModuleLoadData(&m->mod, image);
    if (e != hipSuccess) {
      delete m;
      return hwk::hip_err("hipModuleLoadData", e);
    }
    for (Kernel &k : m->kernels) {
      if (!k.has_geom) continue;
      e = hipModuleGetFunction(&k.fn, m->mod, k.name.c_str());
      if (e != hipSuccess) {
        char *err = hwk::errf("hwk_module_load: kernel %s: %s", k.name.c_str(), hipGetErrorString(e));
        hwk_module_free(m);
        return err;
      }
    }
  }
  *out = m;
  return nullptr;
}

HWK_API void hwk_module_free(hwk_module *m) {
  if (!m) return;
  if (m->mod) (void)hipModuleUnload(m->mod);
  delete m;
}

HWK_API char *hwk_module_kernel_count(hwk_module *m, uint32_t *count) {
  HWK_CHECK(m && count, "hwk_module_kernel_count: null argument");
  *count = (uint32_t)m->kernels.size();
  return nullptr;
}

HWK_API char *hwk_module_kernel_info(hwk_module *m, uint32_t kernel, hwk_kernel_info *out) {
  HWK_CHECK(m && out, "hwk_module_kernel_info: null argument");
  HWK_CHECK(kernel < m->kernels.size(), "hwk_module_kernel_info: kernel %u of %zu", kernel, m->kernels.size());
  const Kernel &k = m->kernels[kernel];
  memset(out, 0, sizeof *out);
  snprintf(out->name, sizeof out->name, "%s", k.name.c_str());
  out->args = (uint32_t)k.args.size();
  out->kernarg_bytes = k.kernarg_bytes;
  out->block = k.has_geom ? k.geom.block : 0;
  out->max_block = k.max_block;
  out->lds_bytes = k.lds_static + (k.has_geom ? k.geom.lds_bytes : 0);
  out->cus = m->dev ? (uint32_t)m->dev->prop.multiProcessorCount : 0;
  out->runnable = k.has_geom ? 1 : 0;
  return nullptr;
}

HWK_API char *hwk_module_kernel_arg(hwk_module *m, uint32_t kernel, uint32_t arg, hwk_kernel_arg *out) {
  HWK_CHECK(m && out, "hwk_module_kernel_arg: null argument");
  HWK_CHECK(kernel < m->kernels.size(), "hwk_module_kernel_arg: kernel %u of %zu", kernel, m->kernels.size());
  const Kernel &k = m->kernels[kernel];
  HWK_CHECK(arg < k.args.size(), "hwk_module_kernel_arg: kernel %s has no argument %u", k.name.c_str(), arg);
  const KArg &a = k.args[arg];
  memset(out, 0, sizeof *out);
  out->index = a.index;
  out->offset = a.offset;
  out->size = a.size;
  out->buffer = a.buffer ? 1 : 0;
  out->nullable = a.nullable ? 1 : 0;
  snprintf(out->name, sizeof out->name, "%s", a.name.c_str());
  snprintf(out->type, sizeof out->type, "%s", type_of(a));
  return nullptr;
}

HWK_API char *hwk_run_new(hwk_module *m, const char *kernel, hwk_run **out) {
  HWK_CHECK(m && kernel && out, "hwk_run_new: null argument");
  HWK_CHECK(m->dev, "hwk_run_new: the module was loaded without a device (inspection only)");
  const Kernel *k = nullptr;
  for (const Kernel &kk : m->kernels)
    if (kk.name == kernel) k = &kk;
  HWK_CHECK(k, "hwk_run_new: no kernel %s", kernel);
  HWK_CHECK(k->has_geom && k->fn, "hwk_run_new: kernel %s has no launch geometry in the code object's manifest", kernel);
  HWK_TRY("hipSetDevice", hipSetDevice(m->dev->index));
  hipEvent_t ev;
  HWK_TRY("hipEventCreateWithFlags", hipEventCreateWithFlags(&ev, hipEventDisableTiming));
  hwk_run *r = new hwk_run();
  r->m = m;
  r->k = k;
  r->args.assign((k->kernarg_bytes + 7) & ~7u, 0);
  r->set.assign(k->args.size(), 0);
  r->done = ev;
  *out = r;
  return nullptr;
}

HWK_API char *hwk_run_set_arg(hwk_run *r, uint32_t index, const void *value, size_t n) {
  HWK_CHECK(r, "hwk_run_set_arg: null run");
  const KArg *a = arg_of(r, index);
  if (!a) return record(r, hwk::errf("hwk_run_set_arg: kernel %s has no argument %u", r->k->name.c_str(), index));
  if (a->buffer)
    return record(r, hwk::errf("hwk_run_set_arg: argument %u (%s) is a buffer", index, a->name.c_str()));
  if (!value || n != a->size)
    return record(r, hwk::errf("hwk_run_set_arg: argument %u (%s) takes %u bytes, got %zu", index, a->name.c_str(),
                               a->size, value ? n : (size_t)0));
  memcpy(r->args.data() + a->offset, value, n);
  r->set[index] = 1;
  return nullptr;
}

HWK_API char *hwk_run_set_buffer_at(hwk_run *r, uint32_t index, hwk_buf *b, size_t off, size_t n) {
  HWK_CHECK(r, "hwk_run_set_buffer_at: null run");
  const KArg *a = arg_of(r, index);
  if (!a) return record(r, hwk::errf("hwk_run_set_buffer: kernel %s has no argument %u", r->k->name.c_str(), index));
  if (!a->buffer)
    return record(r, hwk::errf("hwk_run_set_buffer: argument %u (%s) is not a buffer", index, a->name.c_str()));
  if (!b || !b->ptr) return record(r, hwk::errf("hwk_run_set_buffer: argument %u: nil or closed buffer", index));
  if (b->dev->index != r->m->dev->index)
    return record(r, hwk::errf("hwk_run_set_buffer: argument %u: buffer was not allocated on this device", index));
  if (n == 0 || off > b->size || n > b->size - off)
    return record(r, hwk::errf("hwk_run_set_buffer: argument %u: [%zu, %zu) of a %zu byte buffer", index, off,
                               off + n, b->size));
  if (a->size != 8)
    return record(r, hwk::errf("hwk_run_set_buffer: buffer argument %s has size %u", a->name.c_str(), a->size));
  const uint64_t addr = (uint64_t)(uintptr_t)b->ptr + off;
  memcpy(r->args.data() + a->offset, &addr, 8);
  r->set[index] = 1;
  return nullptr;
}

HWK_API char *hwk_run_set_null(hwk_run *r, uint32_t index) {
  HWK_CHECK(r, "hwk_run_set_null: null run");
  const KArg *a = arg_of(r, index);
  if (!a) return record(r, hwk::errf("hwk_run_set_null: kernel %s has no argument %u", r->k->name.c_str(), index));
  if (!a->buffer || !a->nullable)
    return record(r, hwk::errf("hwk_run_set_null: argument %u (%s) of %s is not an optional buffer", index,
                               a->name.c_str(), r->k->name.c_str()));
  const uint64_t addr = 0;
  memcpy(r->args.data() + a->offset, &addr, 8);
  r->set[index] = 1;
  return nullptr;
}

HWK_API char *hwk_run_set_buffer(hwk_run *r, uint32_t index, hwk_buf *b) {
  HWK_CHECK(r, "hwk_run_set_buffer: null run");
  if (!b) return record(r, hwk::errf("hwk_run_set_buffer: argument %u: nil or closed buffer", index));
  return hwk_run_set_buffer_at(r, index, b, 0, b->size);
}

HWK_API char *hwk_run_err(hwk_run *r) {
  HWK_CHECK(r, "hwk_run_err: null run");
  if (!r->first_err) return nullptr;
  return hwk::errf("%s", r->first_err);
}

HWK_API char *hwk_run_submit(hwk_run *r, void *stream) {
  HWK_CHECK(r, "hwk_run_submit: null run");
  if (r->first_err) return hwk::errf("%s", r->first_err);
  if (r->submitted) {
    const hipError_t q = hipEventQuery(r->done);
    if (q == hipErrorNotReady) return hwk::errf("hwk_run_submit: previous submission of %s is still running", r->k->name.c_str());
    if (q != hipSuccess) return hwk::hip_err("hipEventQuery", q);
  }
  const Kernel &k = *r->k;
  // A buffer argument left unset would reach the kernel as a null address (on the reference's NPU
  // an unused buffer is harmless; here every kernel dereferences its buffers).
  for (size_t i = 0; i < k.args.size(); i++)
    HWK_CHECK(!k.args[i].buffer || r->set[i], "hwk_run_submit: buffer argument %zu (%s) of %s was never set", i,
              k.args[i].name.c_str(), k.name.c_str());
  const hwk_co_geometry &g = k.geom;
  uint64_t gx = g.grid_div;
  if (g.grid_arg != HWK_CO_FIXED_GRID) {
    uint32_t v;
    memcpy(&v, r->args.data() + k.args[g.grid_arg].offset, 4);
    gx = ((uint64_t)v + g.grid_div - 1) / g.grid_div;
  }
  if (g.grid_per_cu) {
    const uint64_t cap = (uint64_t)g.grid_per_cu * (uint64_t)r->m->dev->prop.multiProcessorCount;
    if (gx > cap) gx = cap;
  }
  HWK_CHECK(gx <= 0x7fffffffu, "hwk_run_submit: grid of %llu workgroups", (unsigned long long)gx);
  std::vector<void *> params(k.args.size());
  for (size_t i = 0; i < k.args.size(); i++) params[i] = r->args.data() + k.args[i].offset;
  HWK_TRY("hipSetDevice", hipSetDevice(r->m->dev->index));
  // an empty problem (a grid argument of 0) launches nothing; its fence still completes in stream order
  if (gx > 0)
    HWK_TRY("hipModuleLaunchKernel",
            hipModuleLaunchKernel(k.fn, (uint32_t)gx, 1, 1, g.block, 1, 1, g.lds_bytes, (hipStream_t)stream,
                                  params.empty() ? nullptr : params.data(), nullptr));
  HWK_TRY("hipEventRecord", hipEventRecord(r->done, (hipStream_t)stream));
  r->submitted = true;
  return nullptr;
}

// Polls, so that the wait has a bound: the submission keeps running when the wait gives up (the
// reference's Fence.Wait(ctx) is cancelable the same way, graph.go:144-150).
HWK_API char *hwk_run_wait(hwk_run *r, uint32_t timeout_ms, int *state) {
  HWK_CHECK(r && state, "hwk_run_wait: null argument");
  HWK_CHECK(r->submitted, "hwk_run_wait: %s was never submitted", r->k->name.c_str());
  auto start = std::chrono::steady_clock::now();
  for (;;) {
    const hipError_t e = hipEventQuery(r->done);
    if (e == hipSuccess) {
      *state = HWK_STATE_DONE;
      return nullptr;
    }
    if (e != hipErrorNotReady) return hwk::hip_err("hipEventQuery", e);
    auto ms = std::chrono::duration_cast<std::chrono::milliseconds>(std::chrono::steady_clock::now() - start).count();
    if ((uint64_t)ms >= timeout_ms) {
      *state = HWK_STATE_PENDING;
      return nullptr;
    }
    std::this_thread::sleep_for(std::chrono::microseconds(20));
  }
}

HWK_API char *hwk_run_free(hwk_run *r) {
  if (!r) return nullptr;
  char *err = nullptr;
  if (r->submitted) {
    const hipError_t e = hipEventSynchronize(r->done);
    if (e != hipSuccess) err = hwk::hip_err("hwk_run_free: waiting for the submission", e);
  }
  (void)hipEventDestroy(r->done);
  free(r->first_err);
  delete r;
  return err;
}

}  // extern "C"
