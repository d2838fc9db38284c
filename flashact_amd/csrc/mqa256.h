// Multi-query attention stages shared by the kernels whose attention has the Gemma head layout:
// 8 query heads of 256 dims sharing one K/V head (the pi0.5 action expert and its Gemma-2B
// backbone). Every token of sample b attends to cache rows [0, Lp + Tv) of its layer: the Lp rows
// already in the cache plus the Tv rows this step's QKV stage writes there (no mask among them;
// src/pi05/mk6.cu:312-421 for the expert).
//
// The stages are templates on the kernel's parameter block P, which provides kcache [B][NL][Lmax]
// [256], vtcache [B][NL][256][Lmax], Lp, Tv, B, NL, Lmax and a layout L with NQT (query tiles of
// 16 rows per sample), NKC, and the workspace offsets qf, attp, ml and attn.
#pragma once
#include "engine.h"

namespace fa {
namespace mqa {
using namespace fa::eng;

constexpr int HD = 256, NH = 8, QD = NH * HD;
constexpr int KCH = 128;  // keys per attention chunk
constexpr int QTG = 16;   // query tiles (16 rows) per attention item

// Fragment-ordered Q of sample b: row r = h * Tv + t, dim d -> tile r/16, k-step d/32, lane
// (r % 16) + 16 ((d % 32) / 8), element d % 8.
__host__ __device__ inline uint32_t qf_off(int NQT, int b, int r, int d) {
  return (uint32_t)(((((size_t)b * NQT + (r >> 4)) * 8 + (d >> 5)) * 64 + (r & 15) + 16 * ((d & 31) >> 3)) * 16 +
                    (d & 7) * 2);
}

// ---------------------------------------------------------------- GEMM epilogues
// QKV GEMM epilogue. Output rows: 2048 q (RoPE pairs j, j+128 of each head adjacent), 256 k (pairs
// adjacent), 256 v. RoPE at table row t; q -> fragment-ordered Q, k -> kcache row Lp + t, v ->
// vtcache column Lp + t of layer l.
struct EpiQKV {
  rsrc_t ws, kc, vc;
  const float* rcos;
  const float* rsin;
  uint32_t qf;
  int NQT, Tv, NL, Lmax, Lp, l, split;
  typedef f32x4 Pre;  // cos j0, cos j0+1, sin j0, sin j0+1 of the lane's token
  __device__ Pre pre(int n0, int m) const {
    if (n0 >= 2304) return f32x4{0.f, 0.f, 0.f, 0.f};
    const int t = m % Tv, j0 = ((n0 < 2048 ? n0 : n0 - 2048) >> 1) & 127;
    const f32x2 c = *reinterpret_cast<const f32x2*>(rcos + t * 128 + j0);
    const f32x2 sn = *reinterpret_cast<const f32x2*>(rsin + t * 128 + j0);
    return f32x4{c[0], c[1], sn[0], sn[1]};
  }
  __device__ void operator()(int n0, int m, f32x4 v, f32x4 cs) const {
    const int b = m / Tv, t = m - b * Tv;
    if (n0 >= 2304) {  // v rows: dims n0-2304 .. +3 of key Lp+t
      const int d0 = n0 - 2304;
      const size_t base = (((size_t)b * NL + l) * HD + d0) * Lmax + Lp + t;
#pragma unroll
      for (int i = 0; i < 4; i++) st_b16(vc, (uint32_t)((base + (size_t)i * Lmax) * 2), bf16_bits(v[i]));
      return;
    }
    const int p0 = (n0 < 2048 ? n0 : n0 - 2048) >> 1;  // first of two RoPE pairs
    const int j0 = p0 & 127;
    const float lo0 = v[0] * cs[0] - v[1] * cs[2], hi0 = v[1] * cs[0] + v[0] * cs[2];
    const float lo1 = v[2] * cs[1] - v[3] * cs[3], hi1 = v[3] * cs[1] + v[2] * cs[3];
    const unsigned plo = pack_bf16x2(lo0, lo1), phi = pack_bf16x2(hi0, hi1);
    if (n0 < 2048) {
      const int r = (p0 >> 7) * Tv + t;
      st_b32(ws, qf + qf_off(NQT, b, r, j0), plo);
      st_b32(ws, qf + qf_off(NQT, b, r, j0 + 128), phi);
    } else {
      const size_t row = (((size_t)b * NL + l) * Lmax + Lp + t) * HD;
      st_b32(kc, (uint32_t)((row + j0) * 2), plo);
      st_b32(kc, (uint32_t)((row + j0 + 128) * 2), phi);
    }
  }
};

// ---------------------------------------------------------------- attention partials
// Item (b, kc, qg): keys [128 kc, 128 kc + 128) of sample b against query tiles 16 qg + w + 4 j
// (wave w, j < 4, two tiles per pass). The chunk's K rows and V^T columns are copied
// to LDS once, in MFMA fragment order (64 + 64 fragments). K rows are permuted inside each 32-key
// span so that the S^T accumulators of key tiles (2 sp, 2 sp + 1) are directly the P^T operand of
// k-step sp: tile row 4a + i of key tile 2 sp + kt holds key 32 sp + 8 a + 4 kt + i.
// Keys >= Ltot: S = -inf and their V^T elements are zeroed.
constexpr uint32_t ATT_LDS = 128 * 1024;

template <class P>
__device__ __forceinline__ void stage_att(const P& p, rsrc_t ws, int l) {
  const auto& L = p.L;
  const int w = wave_id(), lane = lane_id(), lr = lane & 15, lq = lane >> 4;
  const int Ltot = p.Lp + p.Tv;
  const int nkc = (Ltot + KCH - 1) / KCH, nqg = (L.NQT + QTG - 1) / QTG;
  const int items = p.B * nkc * nqg;
  const float qscale = 1.4426950408889634f / 16.0f;  // log2(e) / sqrt(256)
#pragma unroll 1
  for (int it = vwg(); it < items; it += NWG) {
    const int qg = it % nqg, rest = it / nqg, kc = rest % nkc, b = rest / nkc;
    const int key0 = kc * KCH, kend = min(key0 + KCH, Ltot);
    const bf16* kb_ = p.kcache + ((size_t)b * p.NL + l) * p.Lmax * HD;
    const bf16* vb_ = p.vtcache + ((size_t)b * p.NL + l) * HD * p.Lmax;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // the previous item's readers are done with LDS
#pragma unroll
    for (int j = 0; j < 32; j++) {
      const int f = w + 4 * j;
      if (f < 64) {  // K fragment (key tile kt8 = f / 8, k-step f % 8)
        const int kt8 = f >> 3, ks = f & 7;
        int key = key0 + 32 * (kt8 >> 1) + 8 * (lr >> 2) + 4 * (kt8 & 1) + (lr & 3);
        if (key >= Ltot) key = 0;
        dma16<true>(kb_ + (size_t)key * HD + ks * 32 + 8 * lq, lds_addr(f * 1024));
      } else {  // V^T fragment (dim tile dt, 32-key span sp)
        const int fv = f - 64, dt = fv >> 2, sp = fv & 3;
        int kg = key0 + 32 * sp + 8 * lq;
        if (kg >= Ltot) kg = 0;
        dma16<true>(vb_ + (size_t)(16 * dt + lr) * p.Lmax + kg, lds_addr(f * 1024));
      }
    }
    unsigned vmask[4][4];  // V^T element masks of keys >= kend
#pragma unroll
    for (int sp = 0; sp < 4; sp++) {
      const int nv = min(max(kend - (key0 + 32 * sp + 8 * lq), 0), 8);
#pragma unroll
      for (int e = 0; e < 4; e++) vmask[sp][e] = nv >= 2 * e + 2 ? 0xffffffffu : (nv == 2 * e + 1 ? 0xffffu : 0u);
    }
    vm_wait<0>();
    __syncthreads();
    // two query tiles per pass (qt, qt + 4): every K / V^T fragment read from LDS feeds 2 MFMAs
#pragma unroll 1
    for (int jp = 0; jp < QTG / 8; jp++) {
      const int qt[2] = {QTG * qg + w + 8 * jp, QTG * qg + w + 8 * jp + 4};
      if (qt[0] >= L.NQT) break;
      const bool has1 = qt[1] < L.NQT;
      u32x4 qf[2][8];
#pragma unroll
      for (int q = 0; q < 2; q++) {
        const int tq = (q == 1 && !has1) ? qt[0] : qt[q];
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
          qf[q][ks] = ldb128<kCpSc1>(ws, (uint32_t)(L.qf + ((((size_t)b * L.NQT + tq) * 8 + ks) * 64 + lane) * 16));
      }
      f32x4 s[2][8];
#pragma unroll
      for (int kt8 = 0; kt8 < 8; kt8++) {
        // the key tile's 8 fragments are read ahead of its 16 MFMAs (read one by one, every MFMA
        // pair would wait out an LDS round trip)
        u32x4 kf[8];
#pragma unroll
        for (int ks = 0; ks < 8; ks++) kf[ks] = lds128((kt8 * 8 + ks) * 1024 + lane * 16);
        __builtin_amdgcn_sched_barrier(0);
        f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 8; ks++) {
          a0 = mfma16(kf[ks], qf[0][ks], a0);
          a1 = mfma16(kf[ks], qf[1][ks], a1);
        }
        __builtin_amdgcn_sched_barrier(0);
        s[0][kt8] = a0;
        s[1][kt8] = a1;
      }
      float mx[2], psum[2];
      u32x4 pb[2][4];
#pragma unroll
      for (int q = 0; q < 2; q++) {
        float m_ = -1e30f;
#pragma unroll
        for (int kt8 = 0; kt8 < 8; kt8++)
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const int key = key0 + 32 * (kt8 >> 1) + 8 * lq + 4 * (kt8 & 1) + i;
            s[q][kt8][i] = key < kend ? s[q][kt8][i] * qscale : -1e30f;
            m_ = fmaxf(m_, s[q][kt8][i]);
          }
        m_ = cols_max(m_);
        float ps = 0.f;
#pragma unroll
        for (int sp = 0; sp < 4; sp++) {
          float pv[8];
#pragma unroll
          for (int kt = 0; kt < 2; kt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
              pv[4 * kt + i] = exp2f(s[q][2 * sp + kt][i] - m_);
              ps += pv[4 * kt + i];
            }
          pb[q][sp] = u32x4{pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3]), pack_bf16x2(pv[4], pv[5]),
                            pack_bf16x2(pv[6], pv[7])};
        }
        ps = cols_sum(ps);
        mx[q] = m_;
        psum[q] = ps;
      }
      // O^T = V^T P^T, one 16-dim tile at a time, stored as soon as it is complete: lane holds
      // O^T[dim 16 dt + 4 lq + i][query row 16 qt + lr]
      bool st[2];
      size_t prow[2];
      float inv[2];
#pragma unroll
      for (int q = 0; q < 2; q++) {
        const int r = 16 * qt[q] + lr;
        st[q] = (q == 0 || has1) && r < NH * p.Tv;
        prow[q] = ((size_t)b * L.NKC + kc) * L.NQT * 16 + r;
        inv[q] = 1.0f / psum[q];
      }
#pragma unroll
      for (int dt = 0; dt < 16; dt++) {
        u32x4 va[4];  // the dim tile's 4 V^T fragments, read ahead of its 8 MFMAs
#pragma unroll
        for (int sp = 0; sp < 4; sp++) va[sp] = lds128((64 + dt * 4 + sp) * 1024 + lane * 16);
        __builtin_amdgcn_sched_barrier(0);
        f32x4 o0 = {0.f, 0.f, 0.f, 0.f}, o1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int sp = 0; sp < 4; sp++) {
#pragma unroll
          for (int e = 0; e < 4; e++) va[sp][e] &= vmask[sp][e];
          o0 = mfma16(va[sp], pb[0][sp], o0);
          o1 = mfma16(va[sp], pb[1][sp], o1);
        }
        if (st[0])
          st_b64(ws, (uint32_t)(L.attp + (prow[0] * HD + 16 * dt + 4 * lq) * 2),
                 u32x2{pack_bf16x2(o0[0] * inv[0], o0[1] * inv[0]), pack_bf16x2(o0[2] * inv[0], o0[3] * inv[0])});
        if (st[1])
          st_b64(ws, (uint32_t)(L.attp + (prow[1] * HD + 16 * dt + 4 * lq) * 2),
                 u32x2{pack_bf16x2(o1[0] * inv[1], o1[1] * inv[1]), pack_bf16x2(o1[2] * inv[1], o1[3] * inv[1])});
      }
#pragma unroll
      for (int q = 0; q < 2; q++)
        if (st[q] && lq == 0) st_b64(ws, (uint32_t)(L.ml + prow[q] * 8), u32x2{as_u32(mx[q]), as_u32(psum[q])});
    }
  }
}

// ---------------------------------------------------------------- combine
// attn[b Tv + t][256 h + d] = sum_c w_c O_c with w_c = l_c 2^(m_c - M) / sum. A wave combines 4
// query rows at once (16 lanes per row, 16 dims per lane); the (m, l) pairs and the partials of up
// to 8 chunks are all in flight together.
template <class P>
__device__ __forceinline__ void stage_comb(const P& p, rsrc_t ws) {
  const auto& L = p.L;
  const int lane = lane_id(), sub = lane >> 4, l16 = lane & 15;
  const int Ltot = p.Lp + p.Tv, nkc = (Ltot + KCH - 1) / KCH;
  const int rows = p.B * NH * p.Tv;
#pragma unroll 1
  for (int R0 = (vwg() * 4 + wave_id()) * 4; R0 < rows; R0 += NWG * 16) {
    const int R = R0 + sub;
    const bool valid = R < rows;
    const int Rc = valid ? R : R0;
    const int b = Rc / (NH * p.Tv), r = Rc - b * NH * p.Tv, h = r / p.Tv, t = r - h * p.Tv;
    const size_t cstride = (size_t)L.NQT * 16;  // rows per chunk
    const size_t row0 = (size_t)b * L.NKC * cstride + r;
    float Mx = -1e30f, den = 0.f;
    f32x4 acc[4] = {};
#pragma unroll 1
    for (int c0 = 0; c0 < nkc; c0 += 8) {
      u32x2 ml[8];
      u32x4 v[8][2];
#pragma unroll
      for (int c = 0; c < 8; c++) {
        const bool ok = c0 + c < nkc;
        const size_t prow = row0 + (size_t)(c0 + c) * cstride;
        ml[c] = ldb64<kCpSc1>(ws, ok ? (uint32_t)(L.ml + prow * 8) : (uint32_t)L.ml);
#pragma unroll
        for (int k = 0; k < 2; k++)
          v[c][k] = ldb128<kCpSc1>(ws, ok ? (uint32_t)(L.attp + (prow * HD + 16 * l16 + 8 * k) * 2) : (uint32_t)L.attp);
      }
#pragma unroll
      for (int c = 0; c < 8; c++) {
        if (c0 + c >= nkc) break;
        const float mc = as_f32(ml[c][0]), lc = as_f32(ml[c][1]);
        const float mn = fmaxf(Mx, mc);
        const float sa = exp2f(Mx - mn), sc = lc * exp2f(mc - mn);
        Mx = mn;
        den = den * sa + sc;
#pragma unroll
        for (int k = 0; k < 2; k++) {
#pragma unroll
          for (int e = 0; e < 2; e++) {
            acc[2 * k + e][0] = acc[2 * k + e][0] * sa + sc * bf_lo(v[c][k][2 * e]);
            acc[2 * k + e][1] = acc[2 * k + e][1] * sa + sc * bf_hi(v[c][k][2 * e]);
            acc[2 * k + e][2] = acc[2 * k + e][2] * sa + sc * bf_lo(v[c][k][2 * e + 1]);
            acc[2 * k + e][3] = acc[2 * k + e][3] * sa + sc * bf_hi(v[c][k][2 * e + 1]);
          }
        }
      }
    }
    if (valid) {
      const float inv = 1.0f / den;
      const int m = b * p.Tv + t;
#pragma unroll
      for (int k = 0; k < 2; k++) {
        const u32x4 o = {pack_bf16x2(acc[2 * k][0] * inv, acc[2 * k][1] * inv),
                         pack_bf16x2(acc[2 * k][2] * inv, acc[2 * k][3] * inv),
                         pack_bf16x2(acc[2 * k + 1][0] * inv, acc[2 * k + 1][1] * inv),
                         pack_bf16x2(acc[2 * k + 1][2] * inv, acc[2 * k + 1][3] * inv)};
        st_b128(ws, (uint32_t)(L.attn + ((size_t)m * QD + h * HD + 16 * l16 + 8 * k) * 2), o);
      }
    }
  }
}

}  // namespace mqa
}  // namespace fa
