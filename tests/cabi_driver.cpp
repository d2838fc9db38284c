// A plain C++ host program that drives the denoise engine through its C ABI only
// (include/flashact_mi355x.h): no Python, no torch. It is the integration a C++ caller writes in
// place of the reference's torch-extension `launch` (src/pi05/binding.cpp:28-68,
// src/molmoact2/binding.cpp:28-83).
//
//   cabi_driver pi05 <dir> NL Lp Tv S Lmax xt_rows
//   cabi_driver ma2  <dir> NL Lk Lkmax Tv adim S xt_rows
//
// Reads the launch's inputs as raw little-endian files from <dir> (names below), uploads them with
// hipMemcpy, allocates and initialises the workspace, enqueues ONE launch on a stream of its own,
// waits, reads the kernel status and writes the updated x_t (and, for pi0.5, both caches) back to
// <dir>/*.out. Prints one line "status=<ABI rc> kstatus=<kernel status> ..." and exits 0 only when
// both are 0.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "flashact_mi355x.h"

namespace {

std::vector<unsigned char> read_file(const std::string& path) {
  FILE* f = std::fopen(path.c_str(), "rb");
  if (!f) {
    std::fprintf(stderr, "cannot open %s\n", path.c_str());
    std::exit(2);
  }
  std::fseek(f, 0, SEEK_END);
  const long n = std::ftell(f);
  std::fseek(f, 0, SEEK_SET);
  std::vector<unsigned char> b((size_t)n);
  if (n > 0 && std::fread(b.data(), 1, (size_t)n, f) != (size_t)n) {
    std::fprintf(stderr, "short read %s\n", path.c_str());
    std::exit(2);
  }
  std::fclose(f);
  return b;
}

void write_file(const std::string& path, const void* p, size_t n) {
  FILE* f = std::fopen(path.c_str(), "wb");
  if (!f || std::fwrite(p, 1, n, f) != n) {
    std::fprintf(stderr, "cannot write %s\n", path.c_str());
    std::exit(2);
  }
  std::fclose(f);
}

#define HIP_OK(x)                                                                         \
  do {                                                                                    \
    hipError_t e_ = (x);                                                                  \
    if (e_ != hipSuccess) {                                                               \
      std::fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));                 \
      std::exit(3);                                                                       \
    }                                                                                     \
  } while (0)

struct Dev {
  std::vector<void*> ptrs;
  // uploads <dir>/<name>.bin and checks its size against the expected element count
  void* up(const std::string& dir, const char* name, size_t expect_bytes) {
    std::vector<unsigned char> h = read_file(dir + "/" + name + ".bin");
    if (h.size() != expect_bytes) {
      std::fprintf(stderr, "%s.bin holds %zu bytes, expected %zu\n", name, h.size(), expect_bytes);
      std::exit(2);
    }
    void* d = nullptr;
    HIP_OK(hipMalloc(&d, h.size()));
    HIP_OK(hipMemcpy(d, h.data(), h.size(), hipMemcpyHostToDevice));
    ptrs.push_back(d);
    return d;
  }
  void* alloc(size_t n) {
    void* d = nullptr;
    HIP_OK(hipMalloc(&d, n));
    ptrs.push_back(d);
    return d;
  }
  ~Dev() {
    for (void* p : ptrs) (void)hipFree(p);
  }
};

template <typename T>
void download(const std::string& path, const void* d, size_t n) {
  std::vector<T> h(n);
  HIP_OK(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost));
  write_file(path, h.data(), n * sizeof(T));
}

int run_pi05(const std::string& dir, int NL, int Lp, int Tv, int S, int Lmax, int xt_rows) {
  const size_t D = 1024, HD = 256, AD = 32, F = 4096;
  Dev dv;
  fa_pi05_args a = {};
  a.weight_dtype = FA_DTYPE_BF16;
  a.w1 = dv.up(dir, "w1", NL * 2560 * D * 2);
  a.wo = dv.up(dir, "wo", NL * D * 2048 * 2);
  a.w2 = dv.up(dir, "w2", NL * 2 * F * D * 2);
  a.w3 = dv.up(dir, "w3", NL * D * F * 2);
  a.mods = (const float*)dv.up(dir, "mods", (size_t)S * NL * 2 * 3 * D * 4);
  a.mod_final = (const float*)dv.up(dir, "mod_final", (size_t)S * 3 * D * 4);
  a.rope_cos = (const float*)dv.up(dir, "rope_cos", (size_t)Tv * 128 * 4);
  a.rope_sin = (const float*)dv.up(dir, "rope_sin", (size_t)Tv * 128 * 4);
  a.w_ain = (const float*)dv.up(dir, "w_ain", D * AD * 4);
  a.b_ain = (const float*)dv.up(dir, "b_ain", D * 4);
  a.w_aout = (const float*)dv.up(dir, "w_aout", AD * D * 4);
  a.b_aout = (const float*)dv.up(dir, "b_aout", AD * 4);
  a.kcache = dv.up(dir, "kcache", (size_t)NL * Lmax * HD * 2);
  a.vtcache = dv.up(dir, "vtcache", (size_t)NL * HD * Lmax * 2);
  a.x_t = (float*)dv.up(dir, "x_t", (size_t)xt_rows * AD * 4);
  a.Lp = Lp;
  a.Lmax = Lmax;
  a.num_steps = S;
  a.Tv = Tv;
  a.num_layers = NL;
  a.batch = 1;
  a.xt_rows = xt_rows;
  a.cache_dtype = FA_DTYPE_BF16;
  a.workspace_bytes = fa_pi05_workspace_bytes(1, Tv, Lmax);
  a.workspace = dv.alloc(a.workspace_bytes);
  hipStream_t s;
  HIP_OK(hipStreamCreate(&s));
  int rc = fa_pi05_workspace_init(a.workspace, a.workspace_bytes, (fa_stream_t)s);
  if (rc == FA_OK) rc = fa_pi05_denoise(&a, (fa_stream_t)s);
  if (rc != FA_OK) std::fprintf(stderr, "fa_pi05_denoise: %s\n", fa_last_error());
  HIP_OK(hipStreamSynchronize(s));
  unsigned kst = 0;
  if (rc == FA_OK) rc = fa_pi05_read_status(a.workspace, &kst);
  download<float>(dir + "/x_t.out", a.x_t, (size_t)xt_rows * AD);
  download<unsigned short>(dir + "/kcache.out", a.kcache, (size_t)NL * Lmax * HD);
  download<unsigned short>(dir + "/vtcache.out", a.vtcache, (size_t)NL * HD * Lmax);
  HIP_OK(hipStreamDestroy(s));
  fa_device_info info;
  int dev = 0;
  HIP_OK(hipGetDevice(&dev));
  const int qrc = fa_device_query(dev, &info);
  std::printf("status=%d kstatus=%u cus=%d xcds=%d coop_max_blocks=%d arch=%s query=%d\n", rc, kst, info.cus,
              info.xcds, info.coop_max_blocks, info.arch, qrc);
  return rc == FA_OK && kst == 0 ? 0 : 1;
}

int run_ma2(const std::string& dir, int NL, int Lk, int Lkmax, int Tv, int adim, int S, int xt_rows) {
  const size_t D = 768, FF = 3072, AD = 32;
  Dev dv;
  fa_ma2_args a = {};
  a.weight_dtype = FA_DTYPE_BF16;
  a.w_qkv = dv.up(dir, "w_qkv", NL * 3 * D * D * 2);
  a.w_so = dv.up(dir, "w_so", NL * D * D * 2);
  a.w_cq = dv.up(dir, "w_cq", NL * D * D * 2);
  a.w_co = dv.up(dir, "w_co", NL * D * D * 2);
  a.w_gu = dv.up(dir, "w_gu", NL * 2 * FF * D * 2);
  a.w_dn = dv.up(dir, "w_dn", NL * D * FF * 2);
  a.b_qkv = (const float*)dv.up(dir, "b_qkv", NL * 3 * D * 4);
  a.b_so = (const float*)dv.up(dir, "b_so", NL * D * 4);
  a.b_cq = (const float*)dv.up(dir, "b_cq", NL * D * 4);
  a.b_co = (const float*)dv.up(dir, "b_co", NL * D * 4);
  a.b_gu = (const float*)dv.up(dir, "b_gu", NL * 2 * FF * 4);
  a.b_dn = (const float*)dv.up(dir, "b_dn", NL * D * 4);
  a.mods = (const float*)dv.up(dir, "mods", (size_t)S * NL * 9 * D * 4);
  a.mod_final = (const float*)dv.up(dir, "mod_final", (size_t)S * 2 * D * 4);
  a.rope_cos = (const float*)dv.up(dir, "rope_cos", (size_t)Tv * 48 * 4);
  a.rope_sin = (const float*)dv.up(dir, "rope_sin", (size_t)Tv * 48 * 4);
  a.w_ain = (const float*)dv.up(dir, "w_ain", D * AD * 4);
  a.b_ain = (const float*)dv.up(dir, "b_ain", D * 4);
  a.w_aout = dv.up(dir, "w_aout", AD * D * 2);
  a.b_aout = (const float*)dv.up(dir, "b_aout", AD * 4);
  a.kctx = dv.up(dir, "kctx", (size_t)NL * Lkmax * D * 2);
  a.vtctx = dv.up(dir, "vtctx", (size_t)NL * D * Lkmax * 2);
  a.x_t = (float*)dv.up(dir, "x_t", (size_t)xt_rows * AD * 4);
  a.Lk = Lk;
  a.Lkmax = Lkmax;
  a.Tv = Tv;
  a.adim = adim;
  a.num_steps = S;
  a.num_layers = NL;
  a.batch = 1;
  a.xt_rows = xt_rows;
  a.workspace_bytes = fa_ma2_workspace_bytes(1, Tv, Lkmax);
  a.workspace = dv.alloc(a.workspace_bytes);
  hipStream_t s;
  HIP_OK(hipStreamCreate(&s));
  int rc = fa_ma2_workspace_init(a.workspace, a.workspace_bytes, (fa_stream_t)s);
  if (rc == FA_OK) rc = fa_ma2_flow(&a, (fa_stream_t)s);
  if (rc != FA_OK) std::fprintf(stderr, "fa_ma2_flow: %s\n", fa_last_error());
  HIP_OK(hipStreamSynchronize(s));
  unsigned kst = 0;
  if (rc == FA_OK) rc = fa_ma2_read_status(a.workspace, &kst);
  download<float>(dir + "/x_t.out", a.x_t, (size_t)xt_rows * AD);
  HIP_OK(hipStreamDestroy(s));
  std::printf("status=%d kstatus=%u\n", rc, kst);
  return rc == FA_OK && kst == 0 ? 0 : 1;
}

}  // namespace

int main(int argc, char** argv) {
  if (fa_abi_version() != FA_ABI_VERSION) {
    std::fprintf(stderr, "ABI mismatch: library %d, header %d\n", fa_abi_version(), FA_ABI_VERSION);
    return 2;
  }
  const std::string mode = argc > 1 ? argv[1] : "";
  if (mode == "pi05" && argc == 9)
    return run_pi05(argv[2], std::atoi(argv[3]), std::atoi(argv[4]), std::atoi(argv[5]), std::atoi(argv[6]),
                    std::atoi(argv[7]), std::atoi(argv[8]));
  if (mode == "ma2" && argc == 10)
    return run_ma2(argv[2], std::atoi(argv[3]), std::atoi(argv[4]), std::atoi(argv[5]), std::atoi(argv[6]),
                   std::atoi(argv[7]), std::atoi(argv[8]), std::atoi(argv[9]));
  std::fprintf(stderr,
               "usage: cabi_driver pi05 <dir> NL Lp Tv S Lmax xt_rows\n"
               "       cabi_driver ma2 <dir> NL Lk Lkmax Tv adim S xt_rows\n");
  return 2;
}
