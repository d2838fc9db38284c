// K/V hand-off into the denoise caches (the `srows > 0` prologue of the reference's pi0.5 launch,
// src/pi05/mk6.cu:258-277; layout notes src/pi05/README.md:91-98). The source is a prefill's
// per-layer cache rows with RoPE applied to interleaved pairs (2d, 2d + 1):
//   kvsrc_k, kvsrc_v [batch][NL][srows][256] bf16, rows [0, Lp) valid.
// The denoise kernels use split-half pairs (d, d + 128) and a transposed V, so
//   kcache[b][l][r][d] = K[2d], kcache[b][l][r][d + 128] = K[2d + 1]    (d < 128)
//   vtcache[b][l][d][r] = V[d]
// for r < Lp. The caches are bf16 like the source (the reference also converts to fp16, which the
// bf16 build does not need). It runs as its own kernel ahead of the denoise launch on the same
// stream; stream order stands in for the reference's grid.sync() after the prologue.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "../../include/flashact_mi355x.h"
#include "fa_device.h"
#include "fa_host.h"

namespace fa {
namespace kvh {

constexpr int HD = 256, RT = 64;  // head dim, rows per tile

// Workgroup = one tile of RT rows of one (sample, layer). K: each thread moves one interleaved
// pair per row (coalesced 4-byte reads, 2-byte writes to two contiguous halves). V: the tile is
// staged in LDS, then written column by column (RT consecutive rows of one dim per 64 threads).
__global__ void __launch_bounds__(256) kv_handoff_kernel(const unsigned short* __restrict__ ksrc,
                                                         const unsigned short* __restrict__ vsrc, int srows,
                                                         unsigned short* __restrict__ kc,
                                                         unsigned short* __restrict__ vt, int NL, int Lp, int Lmax) {
  __shared__ unsigned short tile[RT][HD + 2];
  const int ntile = (Lp + RT - 1) / RT;
  const int bl = blockIdx.x / ntile, r0 = (blockIdx.x % ntile) * RT;  // bl = b * NL + l
  const int nr = min(RT, Lp - r0);
  const size_t src0 = ((size_t)bl * srows + r0) * HD;
  const size_t kdst0 = ((size_t)bl * Lmax + r0) * HD;
  for (int i = threadIdx.x; i < nr * (HD / 2); i += blockDim.x) {
    const int r = i / (HD / 2), d = i % (HD / 2);
    const unsigned pair = *reinterpret_cast<const unsigned*>(ksrc + src0 + (size_t)r * HD + 2 * d);
    kc[kdst0 + (size_t)r * HD + d] = (unsigned short)(pair & 0xffffu);
    kc[kdst0 + (size_t)r * HD + d + HD / 2] = (unsigned short)(pair >> 16);
  }
  for (int i = threadIdx.x; i < nr * (HD / 2); i += blockDim.x) {
    const int r = i / (HD / 2), d = i % (HD / 2);
    const unsigned pair = *reinterpret_cast<const unsigned*>(vsrc + src0 + (size_t)r * HD + 2 * d);
    tile[r][2 * d] = (unsigned short)(pair & 0xffffu);
    tile[r][2 * d + 1] = (unsigned short)(pair >> 16);
  }
  __syncthreads();
  const size_t vdst0 = (size_t)bl * HD * Lmax + r0;
  for (int i = threadIdx.x; i < HD * RT; i += blockDim.x) {
    const int d = i / RT, r = i % RT;
    if (r < nr) vt[vdst0 + (size_t)d * Lmax + r] = tile[r][d];
  }
}

// fp16 caches (the reference's, src/pi05/binding.cpp:6, benchmarks/pi05/eval_numerics.py:83-85)
// -> the bf16 shadow the denoise kernels read: 8 elements per thread and iteration, each
// fp16 -> fp32 (exact) -> bf16 (round to nearest even).
__global__ void __launch_bounds__(256) cache_import_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                           size_t n8) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n8; i += (size_t)gridDim.x * blockDim.x) {
    const u32x4 v = src[i];
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const unsigned w = v[j];
      const float lo = (float)__builtin_bit_cast(_Float16, (unsigned short)(w & 0xffffu));
      const float hi = (float)__builtin_bit_cast(_Float16, (unsigned short)(w >> 16));
      o[j] = pack_bf16x2(lo, hi);
    }
    dst[i] = o;
  }
}

// fp32 -> fp16 bits, round to nearest even (v_cvt_f16_f32)
__device__ __forceinline__ unsigned short f16_bits(float f) { return __builtin_bit_cast(unsigned short, (_Float16)f); }

// The rows a launch wrote, bf16 shadow -> the caller's fp16 caches (round to nearest even):
// kcache rows [r0, r1) and vtcache columns [r0, r1) of every (sample, layer) bl.
__global__ void __launch_bounds__(256) cache_export_kernel(const unsigned short* __restrict__ kb,
                                                           const unsigned short* __restrict__ vb,
                                                           unsigned short* __restrict__ kh,
                                                           unsigned short* __restrict__ vh, int Lmax, int r0,
                                                           int nr) {
  const size_t bl = blockIdx.y;
  const int n = nr * HD;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
    const size_t ko = (bl * Lmax + r0) * HD + i;  // row r0 + i / HD, dim i % HD
    kh[ko] = f16_bits(as_f32((unsigned)kb[ko] << 16));
    const int d = i / nr, r = i - d * nr;
    const size_t vo = (bl * HD + d) * Lmax + r0 + r;
    vh[vo] = f16_bits(as_f32((unsigned)vb[vo] << 16));
  }
}

}  // namespace kvh

size_t pi05_cache_elems(int batch, int num_layers, int Lmax) { return (size_t)batch * num_layers * Lmax * kvh::HD; }

int pi05_cache_import(const fa_pi05_args* a, fa_stream_t stream) {
  using namespace fa::kvh;
  const size_t n = pi05_cache_elems(a->batch, a->num_layers, a->Lmax);  // per cache, a multiple of 8
  unsigned char* sh = static_cast<unsigned char*>(a->cache_shadow);
  const size_t n8 = n / 8;
  const unsigned blocks = (unsigned)std::min<size_t>((n8 + 255) / 256, 8192);
  hipLaunchKernelGGL(cache_import_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     static_cast<const u32x4*>(a->kcache), reinterpret_cast<u32x4*>(sh), n8);
  hipLaunchKernelGGL(cache_import_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                     static_cast<const u32x4*>(a->vtcache), reinterpret_cast<u32x4*>(sh + 2 * n), n8);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return host::fail(FA_ERR_LAUNCH, "fa_pi05_denoise: fp16 cache import: %s", hipGetErrorString(e));
  return FA_OK;
}

int pi05_cache_export(const fa_pi05_args* a, fa_stream_t stream) {
  using namespace fa::kvh;
  const size_t n = pi05_cache_elems(a->batch, a->num_layers, a->Lmax);
  const unsigned short* sh = static_cast<const unsigned short*>(a->cache_shadow);
  const int r0 = a->srows > 0 ? 0 : a->Lp, nr = a->Lp + a->Tv - r0;
  const unsigned bx = (unsigned)std::min((nr * HD + 255) / 256, 64);
  hipLaunchKernelGGL(cache_export_kernel, dim3(bx, (unsigned)(a->batch * a->num_layers)), dim3(256), 0,
                     (hipStream_t)stream, sh, sh + n, static_cast<unsigned short*>(a->kcache),
                     static_cast<unsigned short*>(a->vtcache), a->Lmax, r0, nr);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return host::fail(FA_ERR_LAUNCH, "fa_pi05_denoise: fp16 cache export: %s", hipGetErrorString(e));
  return FA_OK;
}

int pi05_kv_handoff(const fa_pi05_args* a, fa_stream_t stream) {
  using namespace fa::kvh;
  const int ntile = (a->Lp + RT - 1) / RT;
  const size_t blocks = (size_t)a->batch * a->num_layers * ntile;
  if (a->Lp == 0) return FA_OK;
  if (blocks > 0x7fffffffu) return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: hand-off grid too large");
  hipLaunchKernelGGL(kv_handoff_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     static_cast<const unsigned short*>(a->kvsrc_k), static_cast<const unsigned short*>(a->kvsrc_v),
                     a->srows, static_cast<unsigned short*>(a->kcache), static_cast<unsigned short*>(a->vtcache),
                     a->num_layers, a->Lp, a->Lmax);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return host::fail(FA_ERR_LAUNCH, "fa_pi05_denoise: hand-off launch: %s", hipGetErrorString(e));
  return FA_OK;
}

}  // namespace fa

extern "C" size_t fa_pi05_cache_shadow_bytes(int batch, int num_layers, int Lmax) {
  if (batch < 1 || num_layers < 1 || Lmax < 16 || (Lmax & 15)) return 0;
  return 2 * fa::pi05_cache_elems(batch, num_layers, Lmax) * 2;
}
