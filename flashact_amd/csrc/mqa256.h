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
  static constexpr int kRowBytes = 0;
  static constexpr bool kStaged = false;
  rsrc_t ws, kc, vc;
  const float* rcos;
  const float* rsin;
  uint32_t qf;
  int NQT, Tv, NL, Lmax, Lp, l, split;
  float rtv;  // rcp_u(Tv)
  typedef f32x4 Pre;  // cos j0, cos j0+1, sin j0, sin j0+1 of the lane's token
  __device__ Pre pre(int n0, int m) const {
    if (n0 >= 2304) return f32x4{0.f, 0.f, 0.f, 0.f};
    const int t = divmod_u(m, Tv, rtv).r, j0 = ((n0 < 2048 ? n0 : n0 - 2048) >> 1) & 127;
    const f32x2 c = *reinterpret_cast<const f32x2*>(rcos + t * 128 + j0);
    const f32x2 sn = *reinterpret_cast<const f32x2*>(rsin + t * 128 + j0);
    return f32x4{c[0], c[1], sn[0], sn[1]};
  }
  __device__ void operator()(int n0, int m, f32x4 v, f32x4 cs) const {
    const QR bt = divmod_u(m, Tv, rtv);
    const int b = bt.q, t = bt.r;
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
// Item (b, kc, qg): keys [128 kc, 128 kc + 128) of sample b against query tiles 16 qg + w + NWAVE j
// (wave w, j < 16 / NWAVE, two tiles per pass). The chunk's K rows and V^T columns are copied to LDS once,
// by copies of 4 rows x 256 B (one instruction each, the fast global -> LDS pattern) into blocks
// at a pitch of 1040 B, so the 16 rows of an MFMA fragment sit in 16 different blocks and a
// fragment read spreads over all banks:
//   K block (h, s), s = 16 kt + i: dims [128 h, 128 h + 128) of keys x + 32 sp (sp < 4) with
//     x = 8 (i / 4) + 4 kt + i % 4; fragment row i of key tile 2 sp + kt is key 32 sp + x, so the
//     S^T accumulators of key tiles (2 sp, 2 sp + 1) are directly the P^T operand of k-step sp.
//   V^T block y: dims y + 64 rr (rr < 4), the chunk's 128 keys in order.
// Keys >= Ltot: S = -inf and their V^T elements are zeroed.
constexpr uint32_t ATT_PITCH = 1040;
constexpr uint32_t ATT_VB = 64 * ATT_PITCH;       // first V^T block
constexpr uint32_t ATT_LDS = 128 * ATT_PITCH;

// Partial O of a 16-row query tile (tile = (b NKC + kc) NQT + qt): 8 blocks of 1 KB, block dp holds
// dim tiles 2 dp and 2 dp + 1 in MFMA output order. The 16 B at lane (row % 16) + 16 g are dims
// 32 dp + 4 g .. + 3 (8 B), then 32 dp + 16 + 4 g .. + 3 (8 B), of that row, g < 4.
__host__ __device__ inline size_t attp_off(size_t tile, int dp, int lane) {
  return ((tile * 8 + dp) * 64 + lane) * 16;
}

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
    const bool full = kend == key0 + KCH;  // no key of the chunk lies past Ltot
    const bf16* kb_ = p.kcache + ((size_t)b * p.NL + l) * p.Lmax * HD;
    const bf16* vb_ = p.vtcache + ((size_t)b * p.NL + l) * HD * p.Lmax;
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // the previous item's readers are done with LDS
    // q of a pass's two query tiles (qt, qt + 4); a missing second tile repeats the first
    u32x4 qf[2][8];
    auto load_q = [&](int jp) {
      const int q0 = QTG * qg + w + 2 * NWAVE * jp;
      if (q0 >= L.NQT) return;
#pragma unroll
      for (int q = 0; q < 2; q++) {
        const int tq = (q == 1 && q0 + NWAVE >= L.NQT) ? q0 : q0 + NWAVE * q;
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
          qf[q][ks] = ldb128<kCpSc1>(ws, (uint32_t)(L.qf + ((((size_t)b * L.NQT + tq) * 8 + ks) * 64 + lane) * 16));
      }
    };
    // K blocks and the first pass's q, then the V^T blocks, which arrive while the first pass
    // computes S and its softmax (16 copies per wave each; lane: row lq, bytes 16 lr .. + 15).
    // The V^T copies are issued only after the wait for K and q: the compiler's own waits for q
    // count only its own loads, not these copies, so a copy issued after q would be waited for
    // at q's first use.
#pragma unroll
    for (int j = 0; j < 64 / NWAVE; j++) {  // K block (h, s), f = w + NWAVE j
      const int f = w + NWAVE * j, h = f >> 5, sl = f & 31, kt = sl >> 4, i = sl & 15;
      int key = key0 + 32 * lq + 8 * (i >> 2) + 4 * kt + (i & 3);
      if (key >= Ltot) key = 0;
      dma16<true>(kb_ + (size_t)key * HD + 128 * h + 8 * lr, lds_addr(f * ATT_PITCH));
    }
    load_q(0);
    vm_wait<0>();
    __syncthreads();  // K of every wave has landed
#pragma unroll
    for (int j = 0; j < 64 / NWAVE; j++) {  // V^T block y
      const int y = w + NWAVE * j;
      int kg = key0 + 8 * lr;
      if (kg >= Ltot) kg = 0;
      dma16<true>(vb_ + (size_t)(y + 64 * lq) * p.Lmax + kg, lds_addr(ATT_VB + y * ATT_PITCH));
    }
    // two query tiles per pass (qt, qt + NWAVE): every K / V^T fragment read from LDS feeds 2 MFMAs
    constexpr int NPASS = QTG / (2 * NWAVE);
#pragma unroll
    for (int jp = 0; jp < NPASS; jp++) {
      const int qt[2] = {QTG * qg + w + 2 * NWAVE * jp, QTG * qg + w + 2 * NWAVE * jp + NWAVE};
      const bool act = qt[0] < L.NQT;
      if (jp > 0 && !act) break;  // (pass 0 runs its V^T barrier in any case)
      const bool has1 = qt[1] < L.NQT;
      f32x4 s[2][8];
      float mx[2], psum[2];
      u32x4 pb[2][4];
      if (act) {
#pragma unroll
        for (int kt8 = 0; kt8 < 8; kt8++) {
          // the key tile's 8 fragments are read ahead of its 16 MFMAs (read one by one, every MFMA
          // pair would wait out an LDS round trip)
          u32x4 kf[8];
#pragma unroll
          for (int ks = 0; ks < 8; ks++)
            kf[ks] = lds128(((ks >> 2) * 32 + (kt8 & 1) * 16 + lr) * ATT_PITCH + (kt8 >> 1) * 256 + (ks & 3) * 64 +
                            lq * 16);
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
        if (!full) {  // keys past Ltot (K rows copied from key 0): S = -inf
#pragma unroll
          for (int q = 0; q < 2; q++)
#pragma unroll
            for (int kt8 = 0; kt8 < 8; kt8++)
#pragma unroll
              for (int i = 0; i < 4; i++)
                if (key0 + 32 * (kt8 >> 1) + 8 * lq + 4 * (kt8 & 1) + i >= kend) s[q][kt8][i] = -1e30f;
        }
#pragma unroll
        for (int q = 0; q < 2; q++) {
          float m_ = -1e30f;
#pragma unroll
          for (int kt8 = 0; kt8 < 8; kt8++)
#pragma unroll
            for (int i = 0; i < 4; i++) m_ = fmaxf(m_, s[q][kt8][i]);
          m_ = cols_max(m_) * qscale;  // in log2 units
          float ps = 0.f;
#pragma unroll
          for (int sp = 0; sp < 4; sp++) {
            float pv[8];
#pragma unroll
            for (int kt = 0; kt < 2; kt++)
#pragma unroll
              for (int i = 0; i < 4; i++) {
                pv[4 * kt + i] = exp2_w(fmaf(s[q][2 * sp + kt][i], qscale, -m_));
                ps += pv[4 * kt + i];
              }
            pb[q][sp] = u32x4{pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3]), pack_bf16x2(pv[4], pv[5]),
                              pack_bf16x2(pv[6], pv[7])};
          }
          ps = cols_sum(ps);
          mx[q] = m_;
          psum[q] = ps;
        }
      }  // act
      if (jp == 0) {
        vm_wait<0>();
        __syncthreads();  // V^T of every wave has landed
        if (!full && ((kend - key0) & 7)) {
          // Keys [kend, ...) of the 8-key group that straddles kend come from cache rows past
          // Ltot: zero them in V^T so that P = 0 meets a finite value. (Groups wholly past Ltot
          // were copied from key 0 instead.) One thread per dim: the first 256 threads.
          const int d = tid();
          if (d < HD) {
            const int gk = (kend - key0) >> 3, nv = (kend - key0) & 7;
            const uint32_t off = ATT_VB + (d & 63) * ATT_PITCH + (d >> 6) * 256 + gk * 16;
            u32x4 v = lds128(off);
#pragma unroll
            for (int e = 0; e < 4; e++) v[e] &= nv >= 2 * e + 2 ? 0xffffffffu : (nv == 2 * e + 1 ? 0xffffu : 0u);
            *reinterpret_cast<u32x4*>(lds + off) = v;
          }
          __syncthreads();
        }
      }
      if (!act) continue;
      if (jp + 1 < NPASS) load_q(jp + 1);  // the next pass's q, in flight with this pass's P V
      // O^T = V^T P^T, one 16-dim tile at a time: lane holds O^T[dim 16 dt + 4 lq + i][query row
      // 16 qt + lr]. A pair of dim tiles leaves as one 1 KB block of the partial (attp_off).
      bool st[2], rv[2];
      size_t prow[2], tile[2];
      float inv[2];
#pragma unroll
      for (int q = 0; q < 2; q++) {
        const int r = 16 * qt[q] + lr;
        st[q] = q == 0 || has1;
        rv[q] = st[q] && r < NH * p.Tv;
        tile[q] = ((size_t)b * L.NKC + kc) * L.NQT + qt[q];
        prow[q] = tile[q] * 16 + lr;
        inv[q] = 1.0f / psum[q];
      }
      u32x2 ev[2];  // the even dim tile's packed rows, stored with the odd one's
#pragma unroll
      for (int dt = 0; dt < 16; dt++) {
        u32x4 va[4];  // the dim tile's 4 V^T fragments, read ahead of its 8 MFMAs
#pragma unroll
        for (int sp = 0; sp < 4; sp++)
          va[sp] = lds128(ATT_VB + (16 * (dt & 3) + lr) * ATT_PITCH + (dt >> 2) * 256 + sp * 64 + lq * 16);
        __builtin_amdgcn_sched_barrier(0);
        f32x4 o0 = {0.f, 0.f, 0.f, 0.f}, o1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int sp = 0; sp < 4; sp++) {
          o0 = mfma16(va[sp], pb[0][sp], o0);
          o1 = mfma16(va[sp], pb[1][sp], o1);
        }
        const u32x2 w0 = {pack_bf16x2(o0[0] * inv[0], o0[1] * inv[0]), pack_bf16x2(o0[2] * inv[0], o0[3] * inv[0])};
        const u32x2 w1 = {pack_bf16x2(o1[0] * inv[1], o1[1] * inv[1]), pack_bf16x2(o1[2] * inv[1], o1[3] * inv[1])};
        if (dt & 1) {
          if (st[0])
            st_b128(ws, (uint32_t)(L.attp + attp_off(tile[0], dt >> 1, lane)), u32x4{ev[0][0], ev[0][1], w0[0], w0[1]});
          if (st[1])
            st_b128(ws, (uint32_t)(L.attp + attp_off(tile[1], dt >> 1, lane)), u32x4{ev[1][0], ev[1][1], w1[0], w1[1]});
        } else {
          ev[0] = w0;
          ev[1] = w1;
        }
      }
#pragma unroll
      for (int q = 0; q < 2; q++)
        if (rv[q] && lq == 0) st_b64(ws, (uint32_t)(L.ml + prow[q] * 8), u32x2{as_u32(mx[q]), as_u32(psum[q])});
    }
  }
}

// ---------------------------------------------------------------- combine
// attn[b Tv + t][256 h + d] = sum_c w_c O_c with w_c = l_c 2^(m_c - M) / sum. A wave combines 4
// query rows at once (16 lanes per row, 16 dims per lane); the (m, l) pairs and the partials of up
// to 8 chunks are all in flight together. attn is stored in MFMA fragment order (the O projection's
// token operand): the lane's 8 dims c..c+7 (c % 8 = 0) of token m are the 16-byte slot
// (k-quarter (c % 32) / 8, token m % 16) of fragment (m / 16, c / 32).
template <class P>
__device__ __forceinline__ void stage_comb(const P& p, rsrc_t ws) {
  const auto& L = p.L;
  const int lane = lane_id(), sub = lane >> 4, l16 = lane & 15;
  const int dp = l16 >> 1, jh = l16 & 1;  // lane: dims 32 dp + 8 jh .. + 7 and 32 dp + 16 + 8 jh .. + 7
  const int Ltot = p.Lp + p.Tv, nkc = (Ltot + KCH - 1) / KCH;
  const int rows = p.B * NH * p.Tv;
  const float rnt = rcp_u(NH * p.Tv), rtv = rcp_u(p.Tv);
  // with 8 waves, wave-major (consecutive rows on different CUs first), so rows spread over every CU
  const int slot = NWAVE == 8 ? wave_id() * NWG + vwg() : vwg() * NWAVE + wave_id();
#pragma unroll 1
  for (int R0 = slot * 4; R0 < rows; R0 += NWG * NWAVE * 4) {
    const int R = R0 + sub;
    const bool valid = R < rows;
    const int Rc = valid ? R : R0;
    const QR br = divmod_u(Rc, NH * p.Tv, rnt), ht = divmod_u(br.r, p.Tv, rtv);
    const int b = br.q, r = br.r, h = ht.q, t = ht.r;
    const size_t cstride = (size_t)L.NQT * 16;  // rows per chunk
    const size_t row0 = (size_t)b * L.NKC * cstride + r;
    const size_t tile0 = (size_t)b * L.NKC * L.NQT + (r >> 4);
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
          v[c][k] = ldb128<kCpSc1>(ws, ok ? (uint32_t)(L.attp + attp_off(tile0 + (size_t)(c0 + c) * L.NQT, dp,
                                                                          (r & 15) + 16 * (2 * jh + k)))
                                          : (uint32_t)L.attp);
      }
#pragma unroll
      for (int c = 0; c < 8; c++) {
        if (c0 + c >= nkc) break;
        const float mc = as_f32(ml[c][0]), lc = as_f32(ml[c][1]);
        const float mn = fmaxf(Mx, mc);
        const float sa = exp2_w(Mx - mn), sc = lc * exp2_w(mc - mn);
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
      // acc[2 k + e]: dims 32 dp + 16 e + 8 jh + 4 k .. + 3
#pragma unroll
      for (int e = 0; e < 2; e++) {
        const u32x4 o = {pack_bf16x2(acc[e][0] * inv, acc[e][1] * inv), pack_bf16x2(acc[e][2] * inv, acc[e][3] * inv),
                         pack_bf16x2(acc[2 + e][0] * inv, acc[2 + e][1] * inv),
                         pack_bf16x2(acc[2 + e][2] * inv, acc[2 + e][3] * inv)};
        const int c = h * HD + 32 * dp + 16 * e + 8 * jh;
        st_b128(ws, (uint32_t)(L.attn + ((((size_t)(m >> 4) * (QD / 32) + (c >> 5)) * 64 + ((c & 31) >> 3) * 16 + (m & 15)) * 16)), o);
      }
    }
  }
}

}  // namespace mqa
}  // namespace fa
