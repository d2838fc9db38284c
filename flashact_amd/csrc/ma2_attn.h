// MolmoAct2 attention pieces shared by the batched kernel (ma2.hip) and the batch-1 kernel
// (ma2_bs1.hip): head dim 96, LDS fragment layouts, softmax + P V of one 16-query tile.
#pragma once
#include "engine.h"

namespace fa {
namespace ma2att {
using namespace fa::eng;

constexpr int HD = 96;

// LDS fragment layouts (1 KB per fragment, lane = row % 16 + 16 * ((k % 32) / 8), element k % 8):
//   Q   (query tile qt, k-step ks)      rows = tokens
//   K   (key tile kt, k-step ks)        row 4a + i of tile 2 sp + kt = key 32 sp + 8 a + 4 kt + i,
//                                       so the S^T tiles (2 sp, 2 sp + 1) form the P^T operand of span sp
//   V^T (dim tile dt, key span sp)      rows = dims, k = keys 32 sp .. 32 sp + 31 in order
__device__ __forceinline__ uint32_t frag_pos(int row, int k) {
  return (uint32_t)(((row & 15) + 16 * ((k & 31) >> 3)) * 16 + (k & 7) * 2);
}
__device__ __forceinline__ uint32_t kperm_row(int key) {  // key -> (tile * 16 + row) of the K layout
  const int sp = key >> 5, o = key & 31;
  return (uint32_t)((2 * sp + ((o & 7) >> 2)) * 16 + 4 * (o >> 3) + (o & 3));
}

// softmax(S^T) over NKT key tiles (keys 32 (kt/2) + 8 lq + 4 (kt%2) + i < kvalid), P^T operands,
// then O^T = V^T P^T for the 6 dim tiles; returns (max, sum) and O^T (normalised by the sum).
template <int NKT>
__device__ __forceinline__ void attend(const u32x4 (&qf)[3], uint32_t kbase, uint32_t vbase, int kvalid,
                                       const unsigned (&vmask)[NKT / 2][4], float& mx, float& psum, f32x4 (&o)[6]) {
  const int lane = lane_id(), lq = lane >> 4;
  const float qscale = 1.4426950408889634f * 0.10206207261596575f;  // log2(e) / sqrt(96)
  f32x4 s[NKT];
#pragma unroll
  for (int kt = 0; kt < NKT; kt++) {
    u32x4 kf[3];  // read ahead of the key tile's MFMAs
#pragma unroll
    for (int ks = 0; ks < 3; ks++) kf[ks] = lds128(kbase + (kt * 3 + ks) * 1024 + lane * 16);
    __builtin_amdgcn_sched_barrier(0);
    f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 3; ks++) a = mfma16(kf[ks], qf[ks], a);
    s[kt] = a;
  }
  float m_ = -1e30f;
#pragma unroll
  for (int kt = 0; kt < NKT; kt++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int key = 32 * (kt >> 1) + 8 * lq + 4 * (kt & 1) + i;
      s[kt][i] = key < kvalid ? s[kt][i] * qscale : -1e30f;
      m_ = fmaxf(m_, s[kt][i]);
    }
  m_ = cols_max(m_);
  float ps = 0.f;
  u32x4 pb[NKT / 2];
#pragma unroll
  for (int sp = 0; sp < NKT / 2; sp++) {
    float pv[8];
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        pv[4 * kt + i] = exp2_w(s[2 * sp + kt][i] - m_);
        ps += pv[4 * kt + i];
      }
    pb[sp] = u32x4{pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3]), pack_bf16x2(pv[4], pv[5]),
                   pack_bf16x2(pv[6], pv[7])};
  }
  ps = cols_sum(ps);
  const float inv = 1.0f / ps;
#pragma unroll
  for (int dt = 0; dt < 6; dt++) {
    u32x4 va[NKT / 2];  // read ahead of the dim tile's MFMAs
#pragma unroll
    for (int sp = 0; sp < NKT / 2; sp++) va[sp] = lds128(vbase + (dt * (NKT / 2) + sp) * 1024 + lane * 16);
    __builtin_amdgcn_sched_barrier(0);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int sp = 0; sp < NKT / 2; sp++) {
#pragma unroll
      for (int e = 0; e < 4; e++) va[sp][e] &= vmask[sp][e];
      acc = mfma16(va[sp], pb[sp], acc);
    }
    o[dt] = acc * inv;
  }
  mx = m_;
  psum = ps;
}

// All ones for a valid token, zero otherwise, hidden from the optimizer so that `x & mask` stays a
// bitwise AND. Written as `valid ? f(x) : 0`, the selects became branches around f, and the
// compiler's wait analysis (which does not pair branches) then waited at the top of each branch for
// every LDS write issued before it: about a dozen LDS round trips in a row in the self attention.
__device__ __forceinline__ unsigned keep_mask(bool valid) {
  unsigned m = valid ? 0xffffffffu : 0u;
  asm volatile("" : "+v"(m));
  return m;
}
// Elements 4 s .. 4 s + 3 of v as two bf16 pairs, ANDed with a keep_mask.
__device__ __forceinline__ u32x2 pack4(const float (&v)[24], int s, unsigned keep) {
  return u32x2{pack_bf16x2(v[4 * s], v[4 * s + 1]) & keep, pack_bf16x2(v[4 * s + 2], v[4 * s + 3]) & keep};
}

// RMS over the 96 dims of a head held by 4 lanes (xor 16, 32) as 24 values each.
__device__ __forceinline__ void rms96(float (&v)[24]) {
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 24; i++) ss += v[i] * v[i];
  ss = cols_sum(ss);
  const float r = rsqrtf(ss / (float)HD + 1e-6f);
#pragma unroll
  for (int i = 0; i < 24; i++) v[i] *= r;
}

}  // namespace ma2att
}  // namespace fa
