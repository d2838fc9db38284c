// MolmoAct2 action-expert flow loop (src/molmoact2/mk_ma2.cu:258-575): the whole S-step Euler
// loop for a batch of samples in ONE cooperative launch of 256 workgroups x 4 waves, built on the
// stage engine (engine.h). D = 768, 8 heads of 96, F = 3072, action dim 32 (the first `adim`
// dims integrated), t_s = s / S, dt = +1/S.
//
// Per layer (grid barrier after each stage), token m = b * Tv + t of sample b:
//   N_msa  x = embed(x_t) (layer 0) or x += g_mlp * y (down projection); h = adaRMS(x)
//   QKV    [M x 2304] = h W_qkv^T + b_qkv (K split: at small batch the last split of each tile
//          sums the partials, at large batch the consumer stage does)
//   SATT   per (sample, head): per-head RMS of q and k, RoPE (split-half
//          pairs d, d+48 at position t), softmax(q k^T / sqrt(96)) v over the Tv action tokens
//   SO     [M x 768] = attn W_so^T + b_so
//   N_mca  x += g_msa * y; h = adaRMS(x)
//   CQ     [M x 768] = h W_cq^T + b_cq
//   CATT   per (sample, head, 128-key chunk): q = RMS(q) per head, attention over the context
//          keys (kctx rows, vtctx columns of head h) -> normalised partial O + (m, l)
//   COMB   combine of the key chunks -> attn
//   CO     [M x 768] = attn W_co^T + b_co
//   N_mlp  x += g_mca * y; h = adaRMS(x)
//   GU     [M x 6144] = h W_gu^T (rows 2f / 2f+1 = gate f / up f) -> m = silu(g + b_g) (u + b_u)
//          (large batches: a GATE stage applies the activation to the summed partials)
//   DN     [M x 768] = m W_dn^T + b_dn
// then the final norm, action projection and Euler update of x_t[:, :adim].
#include "engine.h"
#include "ma2_attn.h"
#include "../../include/flashact_mi355x.h"
#include "fa_host.h"

namespace fa {
namespace ma2 {
using namespace fa::eng;
using namespace fa::ma2att;

constexpr int D = 768, NH = 8, HD = 96, FF = 3072, AD = 32, QKVN = 3 * D, GUN = 2 * FF;
constexpr int KCH = 128;  // context keys per cross-attention item
constexpr int MAX_TV = 64;
constexpr int MAX_TOKENS = 2048;
constexpr int MAX_KS = FIXUP_MAX_KS;

struct Layout {
  int B, Tv, M, MP, NKC;
  int ks_qkv, ks_d, ks_gu, ks_dn;  // K splits of QKV, the D x D projections, gate/up, down
  int ntiles;  // output tiles of the widest GEMM (one fixup counter each)
  size_t x, xn, attn, h, pqkv, pq, pgu, part, yqkv, yq, yo, cnt, cattp, cml, total;
};

// K split for an [nm x N/BN] tile grid over K: the largest divisor of the 128-wide k steps that
// keeps the item count within one pass of the 256 workgroups.
__host__ __device__ inline int pick_ks(int nm, int nn, int K) {
  const int steps = K / 128;
  int best = 1;
  for (int ks = 1; ks <= steps && ks <= MAX_KS; ks++)
    if (steps % ks == 0 && nm * nn * ks <= NWG) best = ks;
  return best;
}

// BM x BN tiles for every GEMM but gate/up, BM x BNG for gate/up.
__host__ __device__ inline Layout layout(int B, int Tv, int Lkmax, int BM, int BN, int BNG) {
  Layout L;
  L.B = B;
  L.Tv = Tv;
  L.M = B * Tv;
  L.MP = (L.M + BM - 1) / BM * BM;
  L.NKC = (Lkmax + KCH - 1) / KCH;
  const int nm = L.MP / BM;
  L.ks_qkv = pick_ks(nm, QKVN / BN, D);
  L.ks_d = pick_ks(nm, D / BN, D);
  L.ks_gu = pick_ks(nm, GUN / BNG, D);
  L.ks_dn = pick_ks(nm, D / BN, FF);
  const int ks_part = L.ks_d > L.ks_dn ? L.ks_d : L.ks_dn;
  size_t o = kWsDataBase;  // control words, epoch flags and the fixup counters below
  auto take = [&](size_t n) {
    const size_t r = o;
    o += (n + 255) / 256 * 256;
    return r;
  };
  L.x = take((size_t)L.MP * D * 4);
  L.xn = take((size_t)L.MP * D * 2);
  L.attn = take((size_t)L.MP * D * 2);
  L.h = take((size_t)L.MP * FF * 2);
  L.pqkv = take((size_t)L.ks_qkv * L.MP * QKVN * 4);
  L.pq = take((size_t)L.ks_d * L.MP * D * 4);
  L.pgu = take((size_t)L.ks_gu * L.MP * GUN * 4);
  L.part = take((size_t)ks_part * L.MP * D * 4);
  L.yqkv = take((size_t)L.MP * QKVN * 4);
  L.yq = take((size_t)L.MP * D * 4);
  L.yo = take((size_t)L.MP * D * 4);
  L.ntiles = nm * (GUN / BNG);
  L.cnt = kWsCounters;  // fixed: never moves with the shape, so a reused workspace keeps them zero
  L.cattp = take((size_t)B * NH * L.NKC * MAX_TV * HD * 2);
  L.cml = take((size_t)B * NH * L.NKC * MAX_TV * 8);
  L.total = o;
  return L;
}
constexpr uint32_t OFF_CTRL = 0, OFF_FLAGS = 1024;

struct Params {
  const bf16 *w_qkv, *w_so, *w_cq, *w_co, *w_gu, *w_dn;
  const float *b_qkv, *b_so, *b_cq, *b_co, *b_gu, *b_dn;
  const float *mods, *mod_final, *rope_cos, *rope_sin, *w_ain, *b_ain;
  const bf16* w_aout;
  const float* b_aout;
  const bf16* kctx;   // [B][NL][Lkmax][768]
  const bf16* vtctx;  // [B][NL][768][Lkmax]
  float* x_t;         // [B][xt_rows][32]
  unsigned long long* stage_cycles;
  unsigned char* ws;
  Layout L;
  int NL, Lk, Lkmax, Tv, adim, S, B, xt_rows;
};

// Byte offset of element (token m, column c) of a [M][K] bf16 activation stored in MFMA fragment order
// (the GEMMs' token operand): fragment (m / 16, c / 32) of 1 KB, 16-byte slot (k-quarter (c % 32) / 8,
// token m % 16), element c % 8.
__device__ __forceinline__ uint32_t afrag(int m, int c, int K) {
  return (uint32_t)((((size_t)(m >> 4) * (K / 32) + (c >> 5)) * 64 + ((c & 31) >> 3) * 16 + (m & 15)) * 16 + (c & 7) * 2);
}

struct FinBias {  // y[m][n..n+3] = sum + bias (fp32)
  rsrc_t ws;
  uint32_t off;
  int N;
  const float* bias;
  __device__ void operator()(int n, int m, f32x4 v) const {
    st_b128(ws, off + (uint32_t)(((size_t)m * N + n) * 4), as_u32x4(v + *reinterpret_cast<const f32x4*>(bias + n)));
  }
};

struct FinSiluGate {  // columns 2f, 2f+1 = gate f, up f -> h[m][f] = silu(g + b_g) (u + b_u) (bf16)
  rsrc_t ws;
  uint32_t off;
  const float* bias;
  __device__ void operator()(int n, int m, f32x4 v) const {
    const f32x4 b = *reinterpret_cast<const f32x4*>(bias + n);
    st_b32(ws, off + (uint32_t)(((size_t)m * FF + (n >> 1)) * 2),
           pack_bf16x2(silu(v[0] + b[0]) * (v[1] + b[1]), silu(v[2] + b[2]) * (v[3] + b[3])));
  }
};

// Gate/up GEMM without a K split: rows 2f, 2f+1 = gate f, up f -> h[m][f] = silu(g + b_g) (u + b_u)
// straight from the tile (bf16, whole 128-byte rows through LDS), instead of fp32 partials, a
// separate gate stage and its grid barrier: batch 16 43.4 -> 40.9 ms per launch (stored in place,
// 4 bytes into each of 16 rows per instruction, the fused stage took 18.5 instead of 13.2 µs).
struct EpiSiluGate {
  static constexpr int kRowBytes = 4;
  static constexpr bool kStaged = true;
  rsrc_t ws;
  uint32_t off;
  const float* bias;
  int split;
  typedef f32x4 Pre;  // biases of features n..n+3, fetched before the tile's first copies
  __device__ Pre pre(int n, int) const { return *reinterpret_cast<const f32x4*>(bias + n); }
  __device__ u32x4 pack(int, f32x4 v, f32x4 b) const {
    return u32x4{pack_bf16x2(silu(v[0] + b[0]) * (v[1] + b[1]), silu(v[2] + b[2]) * (v[3] + b[3])), 0u, 0u, 0u};
  }
  __device__ uint32_t row_off(int m, int n0) const { return off + (uint32_t)(((size_t)m * FF + (n0 >> 1)) * 2); }
};

struct EpiPartN : NoPre {  // fp32 partial sums [split][MP][N] (summed by the consumer stage)
  static constexpr int kRowBytes = 16;
  static constexpr bool kStaged = true;
  rsrc_t ws;
  uint32_t off;
  int MP, N, split;
  __device__ u32x4 pack(int, f32x4 v) const { return as_u32x4(v); }
  __device__ uint32_t row_off(int m, int n0) const { return off + (uint32_t)((((size_t)split * MP + m) * N + n0) * 4); }
};

// acc[q] += sum over the `ks` fp32 partial rows [s][MP][N] of row m, columns c[q]..c[q]+3; PB
// partials (NC x PB 16-byte loads) are in flight per round trip.
template <int NC, int PB>
__device__ __forceinline__ void add_parts(rsrc_t ws, size_t base, int ks, int MP, int N, int m, const int (&c)[NC],
                                          f32x4 (&acc)[NC]) {
#pragma unroll 1
  for (int s0 = 0; s0 < ks; s0 += PB) {
    u32x4 v[PB][NC];
#pragma unroll
    for (int j = 0; j < PB; j++) {
      const int sp = s0 + j < ks ? s0 + j : ks - 1;
#pragma unroll
      for (int q = 0; q < NC; q++) v[j][q] = ldb128<kCpSc1>(ws, (uint32_t)(base + (((size_t)sp * MP + m) * N + c[q]) * 4));
    }
#pragma unroll
    for (int j = 0; j < PB; j++)
      if (s0 + j < ks)
#pragma unroll
        for (int q = 0; q < NC; q++) acc[q] += as_f32x4(v[j][q]);
  }
}

// The input y of a residual / attention stage: FIX = the finished projection (bias included, one
// buffer), otherwise the sum of its `ks` K-split partials plus the bias.
struct YSrc {
  size_t fin;    // [MP][N] finished values (FIX)
  size_t parts;  // [ks][MP][N] partials (otherwise)
  int ks, N;
  const float* bias;
};

// ---------------------------------------------------------------- norm rows
// One wave per token row; lane holds columns 4 lane + 256 k + i (k < 3). MODE 0: x = embed(x_t);
// MODE 1: x += gate * y (the previous projection, see YSrc); MODE 2: as 1, then the final norm,
// the action projection and the Euler update of x_t[:, :adim].
template <int MODE, bool FIX>
__device__ __forceinline__ void stage_norm(const Params& p, rsrc_t ws, rsrc_t xtr, const YSrc& y, const float* gate,
                                           const float* scale, const float* shift, float dt) {
  const Layout& L = p.L;
  const int lane = lane_id();
#pragma unroll 1
  for (int m = wave_id() * NWG + (int)blockIdx.x; m < L.M; m += NWG * 4) {
    const int b = m / p.Tv, t = m - b * p.Tv;
    const uint32_t xto = (uint32_t)(((size_t)b * p.xt_rows + t) * AD * 4);
    f32x4 x[3];
    if (MODE == 0) {
      const float xl = lane < AD ? ldbf32<kCpSc1>(xtr, xto + lane * 4) : 0.f;
      float xa[AD];
#pragma unroll
      for (int a = 0; a < AD; a++) xa[a] = __shfl(xl, a, 64);
#pragma unroll
      for (int k = 0; k < 3; k++) {
        const int d = 4 * lane + 256 * k;
        const f32x4 bb = *reinterpret_cast<const f32x4*>(p.b_ain + d);
#pragma unroll
        for (int i = 0; i < 4; i++) {
          float s = bb[i];
#pragma unroll
          for (int q = 0; q < 8; q++) {
            const f32x4 wv = *reinterpret_cast<const f32x4*>(p.w_ain + (d + i) * AD + 4 * q);
#pragma unroll
            for (int e = 0; e < 4; e++) s = fmaf(wv[e], xa[4 * q + e], s);
          }
          x[k][i] = s;
        }
      }
    } else {
      u32x4 xo[3];
      int cols[3];
      f32x4 yv[3];
#pragma unroll
      for (int k = 0; k < 3; k++) {
        cols[k] = 4 * lane + 256 * k;
        xo[k] = ldb128<kCpSc1>(ws, (uint32_t)(L.x + ((size_t)m * D + cols[k]) * 4));
      }
      if (FIX) {
#pragma unroll
        for (int k = 0; k < 3; k++) yv[k] = as_f32x4(ldb128<kCpSc1>(ws, (uint32_t)(y.fin + ((size_t)m * D + cols[k]) * 4)));
      } else {
#pragma unroll
        for (int k = 0; k < 3; k++) yv[k] = *reinterpret_cast<const f32x4*>(y.bias + cols[k]);
        add_parts<3, 4>(ws, y.parts, y.ks, L.MP, D, m, cols, yv);
      }
#pragma unroll
      for (int k = 0; k < 3; k++) x[k] = as_f32x4(xo[k]) + *reinterpret_cast<const f32x4*>(gate + cols[k]) * yv[k];
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < 3; k++) ss += x[k][0] * x[k][0] + x[k][1] * x[k][1] + x[k][2] * x[k][2] + x[k][3] * x[k][3];
    const float rr = rsqrtf(wave_sum(ss) / (float)D + 1e-6f);
    f32x4 h[3];
#pragma unroll
    for (int k = 0; k < 3; k++) {
      const int d = 4 * lane + 256 * k;
      const f32x4 sc = *reinterpret_cast<const f32x4*>(scale + d);
      const f32x4 sh = *reinterpret_cast<const f32x4*>(shift + d);
#pragma unroll
      for (int i = 0; i < 4; i++) h[k][i] = x[k][i] * rr * (1.0f + sc[i]) + sh[i];
    }
    if (MODE != 2) {
#pragma unroll
      for (int k = 0; k < 3; k++) {
        const int d = 4 * lane + 256 * k;
        st_b128(ws, (uint32_t)(L.x + ((size_t)m * D + d) * 4), as_u32x4(x[k]));
        // xn in fragment order, whole 16-byte slots: lanes (2j, 2j + 1) hold columns 8j .. 8j + 7 of
        // this k; the even lane stores the slot for even k, the odd lane for odd k
        const unsigned lo = pack_bf16x2(h[k][0], h[k][1]), hi = pack_bf16x2(h[k][2], h[k][3]);
        const unsigned plo = swap_adj(lo), phi = swap_adj(hi);
        if ((lane & 1) == (k & 1))
          st_b128(ws, (uint32_t)L.xn + afrag(m, d & ~7, D), (lane & 1) ? u32x4{plo, phi, lo, hi} : u32x4{lo, hi, plo, phi});
      }
    } else {
      float acc = 0.f;  // lane a < adim ends with v[a]
#pragma unroll 1
      for (int a = 0; a < p.adim; a++) {
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < 3; k++) {
          const u32x2 wv = *reinterpret_cast<const u32x2*>(p.w_aout + (size_t)a * D + 4 * lane + 256 * k);
          s += bf_lo(wv[0]) * h[k][0] + bf_hi(wv[0]) * h[k][1] + bf_lo(wv[1]) * h[k][2] + bf_hi(wv[1]) * h[k][3];
        }
        s = wave_sum(s);
        if (lane == a) acc = s;
      }
      if (lane < p.adim) {
        const float xo = ldbf32<kCpSc1>(xtr, xto + lane * 4);
        __builtin_amdgcn_raw_buffer_store_b32(as_u32(xo + dt * (acc + p.b_aout[lane])), xtr, xto + lane * 4, 0,
                                              kCpSc1);
      }
    }
  }
}

// ---------------------------------------------------------------- gate/up activation
// h[m][f] = silu(sum g + b_g) * (sum u + b_u); rows 2f / 2f+1 of the partials are gate f / up f.
// Lane columns c = 4 lane + 256 k (g, u of f = c/2, c/2 + 1), 8 columns per round trip.
__device__ __forceinline__ void stage_gate(const Params& p, rsrc_t ws, int l) {
  const Layout& L = p.L;
  const int lane = lane_id();
  const float* bg = p.b_gu + (size_t)l * GUN;
#pragma unroll 1
  for (int m = wave_id() * NWG + (int)blockIdx.x; m < L.M; m += NWG * 4) {
#pragma unroll 1
    for (int k0 = 0; k0 < GUN / 256; k0 += 8) {
      int cols[8];
      f32x4 v[8];
#pragma unroll
      for (int k = 0; k < 8; k++) {
        cols[k] = 4 * lane + 256 * (k0 + k);
        v[k] = *reinterpret_cast<const f32x4*>(bg + cols[k]);
      }
      add_parts<8, 2>(ws, L.pgu, L.ks_gu, L.MP, GUN, m, cols, v);
#pragma unroll
      for (int k = 0; k < 8; k++)
        st_b32(ws, (uint32_t)(L.h + ((size_t)m * FF + (cols[k] >> 1)) * 2),
               pack_bf16x2(silu(v[k][0]) * v[k][1], silu(v[k][2]) * v[k][3]));
    }
  }
}

// ---------------------------------------------------------------- attention pieces
// The lane's 24 of the 96 columns c0[t] .. c0[t] + 95 of row m of the projection y (finished, or
// partials + bias), for each of NT bases: v[t][4 s + i] = column c0[t] + 16 s + 4 g4 + i (g4 = lane / 16),
// so the four lanes of a row read 64 contiguous bytes per load (with 24 consecutive columns per lane
// they were 96 bytes apart, and a wave's 1 KB load touched about seven 128-byte lines per KB), and
// the RoPE partners j, j + 48 sit in elements 4 s + i, 4 s + 12 + i of one lane.
template <int NT, bool FIX>
__device__ __forceinline__ void load24(rsrc_t ws, const YSrc& y, int MP, int m, const int (&c0)[NT],
                                       float (&v)[NT][24]) {
  const int g4 = lane_id() >> 4;
  int cols[6 * NT];
  f32x4 acc[6 * NT];
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int q = 0; q < 6; q++) cols[6 * t + q] = c0[t] + 16 * q + 4 * g4;
  if (FIX) {
    u32x4 r[6 * NT];
#pragma unroll
    for (int i = 0; i < 6 * NT; i++) r[i] = ldb128<kCpSc1>(ws, (uint32_t)(y.fin + ((size_t)m * y.N + cols[i]) * 4));
#pragma unroll
    for (int i = 0; i < 6 * NT; i++) acc[i] = as_f32x4(r[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 6 * NT; i++) acc[i] = *reinterpret_cast<const f32x4*>(y.bias + cols[i]);
    add_parts<6 * NT, (NT == 1 ? 6 : 1)>(ws, y.parts, y.ks, MP, y.N, m, cols, acc);
  }
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int q = 0; q < 6; q++)
#pragma unroll
      for (int i = 0; i < 4; i++) v[t][4 * q + i] = acc[6 * t + q][i];
}

// Self attention of (sample b, head h) over its Tv action tokens. Wave w prepares tokens
// 16w..16w+15 (lane: token 16w + l%16, dims 16 s + 4 (l/16) + i, s < 6, i < 4) into the LDS Q/K/V^T fragments
// (zeros past Tv), then attends with query tile w.
constexpr uint32_t S_Q = 0, S_K = 12 * 1024, S_V = 24 * 1024;

template <bool FIX>
__device__ __forceinline__ void stage_satt(const Params& p, rsrc_t ws, const YSrc& y) {
  const Layout& L = p.L;
  const int w = wave_id(), lane = lane_id(), lr = lane & 15, g4 = lane >> 4;
#pragma unroll 1
  for (int it = vwg(); it < p.B * NH; it += NWG) {
    const int b = it / NH, h = it - b * NH;
    const int tau = 16 * w + lr;
    const bool tv = tau < p.Tv;
    const int m = b * p.Tv + (tv ? tau : 0);
    float qkv[3][24];
    {
      const int c0 = HD * h;
      const int cs[3] = {c0, D + c0, 2 * D + c0};
      load24<3, FIX>(ws, y, L.MP, m, cs, qkv);
    }
    float (&q)[24] = qkv[0];
    float (&k)[24] = qkv[1];
    float (&v)[24] = qkv[2];
    rms96(q);
    rms96(k);
    // RoPE on split-half pairs (j, j + 48) = elements (4 s + i, 4 s + 12 + i) of the lane, s < 3
    const float* rc = p.rope_cos + (tv ? tau : 0) * 48;
    const float* rs = p.rope_sin + (tv ? tau : 0) * 48;
#pragma unroll
    for (int s = 0; s < 3; s++) {
      const f32x4 c4 = *reinterpret_cast<const f32x4*>(rc + 16 * s + 4 * g4);
      const f32x4 s4 = *reinterpret_cast<const f32x4*>(rs + 16 * s + 4 * g4);
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int a = 4 * s + i, bb = a + 12;
        const float q0 = q[a], q1 = q[bb], k0 = k[a], k1 = k[bb];
        q[a] = q0 * c4[i] - q1 * s4[i];
        q[bb] = q0 * s4[i] + q1 * c4[i];
        k[a] = k0 * c4[i] - k1 * s4[i];
        k[bb] = k0 * s4[i] + k1 * c4[i];
      }
    }
    __syncthreads();  // the previous item's readers are done with LDS
    unsigned short* lq16 = reinterpret_cast<unsigned short*>(lds);
    // q and k rows: each 4-dim group of the lane is half an 8-dim fragment slot (8-byte writes); V^T
    // is transposed, one element per write
    const uint32_t kr = kperm_row(tau);
    const unsigned keep = keep_mask(tv);
#pragma unroll
    for (int s = 0; s < 6; s++) {
      const int d = 16 * s + 4 * g4;
      const u32x2 qs = pack4(q, s, keep);
      const u32x2 ks = pack4(k, s, keep);
      *reinterpret_cast<u32x2*>(lds + S_Q + ((tau >> 4) * 3 + (d >> 5)) * 1024 + frag_pos(tau, d)) = qs;
      *reinterpret_cast<u32x2*>(lds + S_K + ((kr >> 4) * 3 + (d >> 5)) * 1024 + frag_pos(kr, d)) = ks;
    }
#pragma unroll
    for (int s = 0; s < 6; s++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int d = 16 * s + 4 * g4 + i;
        lq16[(S_V + ((d >> 4) * 2 + (tau >> 5)) * 1024 + frag_pos(d, tau)) >> 1] = (unsigned short)(bf16_bits(v[4 * s + i]) & keep);
      }
    __syncthreads();
    if (16 * w < p.Tv) {
      u32x4 qf[3];
#pragma unroll
      for (int ks = 0; ks < 3; ks++) qf[ks] = lds128(S_Q + (w * 3 + ks) * 1024 + lane * 16);
      unsigned vmask[2][4];
#pragma unroll
      for (int sp = 0; sp < 2; sp++)
#pragma unroll
        for (int e = 0; e < 4; e++) vmask[sp][e] = 0xffffffffu;  // keys past Tv hold zeros
      float mx, ps;
      f32x4 o[6];
      attend<4>(qf, S_K, S_V, p.Tv, vmask, mx, ps, o);
      const int t = 16 * w + lr;
      if (t < p.Tv) {
        const int mo = b * p.Tv + t;
#pragma unroll
        for (int dt = 0; dt < 6; dt++)
          st_b64(ws, (uint32_t)L.attn + afrag(mo, HD * h + 16 * dt + 4 * g4, D),
                 u32x2{pack_bf16x2(o[dt][0], o[dt][1]), pack_bf16x2(o[dt][2], o[dt][3])});
      }
    }
  }
}

// Cross attention item (b, h, kc): context keys [128 kc, 128 kc + 128) of head h. The chunk's K
// rows and V^T columns are copied to LDS (24 + 24 fragments); wave i of the item prepares the query
// rows 16 i .. 16 i + 15 (sum of the CQ partials + b_cq, per-head RMS) and attends with them. With
// Tv <= 32 an item needs two waves, and waves 0-1 and 2-3 run two items side by side, each in its
// own C_ITEM bytes of LDS; otherwise all four waves run one item. The context is a launch input, so
// the copies of a workgroup's first trip are issued inside the grid barrier before the stage
// (`catt_prefetch`), under the wait for the CQ stage (batch 16: CATT 11.2 -> 7.5 us per layer).
constexpr uint32_t C_Q = 0, C_K = 12 * 1024, C_V = 36 * 1024, C_ITEM = 60 * 1024;
static_assert(2 * C_ITEM <= 136 * 1024, "two cross-attention items fit the attention LDS");

// Copies fragments f0, f0 + fs, ... (< 48) of cross-attention item it (its context keys' K rows and
// V^T columns) into the item's LDS slot at cb.
__device__ __forceinline__ void catt_copy(const Params& p, int l, int it, uint32_t cb, int f0, int fs) {
  const int lane = lane_id(), lr = lane & 15, g4 = lane >> 4;
  const int nkc = (p.Lk + KCH - 1) / KCH;
  const int kc = it % nkc, rest = it / nkc, h = rest % NH, b = rest / NH;
  const int key0 = kc * KCH;
  const bf16* kb_ = p.kctx + ((size_t)b * p.NL + l) * p.Lkmax * D + HD * h;
  const bf16* vb_ = p.vtctx + (((size_t)b * p.NL + l) * D + HD * h) * p.Lkmax;
#pragma unroll 1
  for (int f = f0; f < 48; f += fs) {
    if (f < 24) {  // K fragment (key tile kt = f / 3, k-step f % 3)
      const int kt = f / 3, ks = f - 3 * kt;
      int key = key0 + 32 * (kt >> 1) + 8 * (lr >> 2) + 4 * (kt & 1) + (lr & 3);
      if (key >= p.Lk) key = 0;
      dma16<false>(kb_ + (size_t)key * D + ks * 32 + 8 * g4, lds_addr(cb + C_K + f * 1024));
    } else {  // V^T fragment (dim tile dt, span sp)
      const int fv = f - 24, dt = fv >> 2, sp = fv & 3;
      int kg = key0 + 32 * sp + 8 * g4;
      if (kg >= p.Lk) kg = 0;
      dma16<false>(vb_ + (size_t)(16 * dt + lr) * p.Lkmax + kg, lds_addr(cb + C_V + fv * 1024));
    }
  }
}

// The first trip's copies of every item slot, issued by waves 1-3 inside the grid barrier that
// precedes the cross attention (the context does not depend on anything the barrier publishes).
__device__ __forceinline__ void catt_prefetch(const Params& p, int l) {
  const int items = p.B * NH * ((p.Lk + KCH - 1) / KCH);
  const int nslot = p.Tv <= 32 ? 2 : 1;
#pragma unroll 1
  for (int slot = 0; slot < nslot; slot++) {
    const int it = vwg() + NWG * slot;
    if (it < items) catt_copy(p, l, it, slot * C_ITEM, wave_id() - 1, 3);
  }
}

template <bool FIX>
__device__ __forceinline__ void stage_catt(const Params& p, rsrc_t ws, int l, const YSrc& y, bool pre) {
  const Layout& L = p.L;
  const int w = wave_id(), lane = lane_id(), lr = lane & 15, g4 = lane >> 4;
  const int nkc = (p.Lk + KCH - 1) / KCH, items = p.B * NH * nkc;
  const int wpi = p.Tv <= 32 ? 2 : 4;     // waves per item
  const int slot = w / wpi, wi = w % wpi;  // item slot of this wave, its index within the item
  const uint32_t cb = slot * C_ITEM;
#pragma unroll 1
  for (int it0 = vwg(); it0 < items; it0 += NWG * (4 / wpi)) {  // every wave takes the same trips
    const int it = it0 + NWG * slot;
    const bool act = it < items;
    const int kc = it % nkc, rest = it / nkc, h = rest % NH, b = rest / NH;
    const int kvalid = min(KCH, p.Lk - kc * KCH);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();  // the previous item's readers are done with LDS
    if (act) {
      if (!pre || it0 != vwg()) catt_copy(p, l, it, cb, wi, wpi);  // pre: the first trip's are in flight
      // query rows of this wave
      const int tau = 16 * wi + lr;
      const bool tv = tau < p.Tv;
      float qq[1][24];
      {
        const int cs[1] = {HD * h};
        load24<1, FIX>(ws, y, L.MP, b * p.Tv + (tv ? tau : 0), cs, qq);
      }
      float (&q)[24] = qq[0];
      rms96(q);
      const unsigned keep = keep_mask(tv);
#pragma unroll
      for (int s = 0; s < 6; s++) {  // element 4 s + i = dim 16 s + 4 g4 + i: half a fragment slot each
        const int d = 16 * s + 4 * g4;
        const u32x2 qs = pack4(q, s, keep);
        *reinterpret_cast<u32x2*>(lds + cb + C_Q + ((tau >> 4) * 3 + (d >> 5)) * 1024 + frag_pos(tau, d)) = qs;
      }
    }
    unsigned vmask[4][4];
#pragma unroll
    for (int sp = 0; sp < 4; sp++) {
      const int nv = min(max(kvalid - (32 * sp + 8 * g4), 0), 8);
#pragma unroll
      for (int e = 0; e < 4; e++) vmask[sp][e] = nv >= 2 * e + 2 ? 0xffffffffu : (nv == 2 * e + 1 ? 0xffffu : 0u);
    }
    vm_wait<0>();
    __syncthreads();
    if (act && 16 * wi < p.Tv) {
      u32x4 qf[3];
#pragma unroll
      for (int ks = 0; ks < 3; ks++) qf[ks] = lds128(cb + C_Q + (wi * 3 + ks) * 1024 + lane * 16);
      float mx, ps;
      f32x4 o[6];
      attend<8>(qf, cb + C_K, cb + C_V, kvalid, vmask, mx, ps, o);
      const int t = 16 * wi + lr;
      if (t < p.Tv) {
        const size_t prow = (((size_t)b * NH + h) * L.NKC + kc) * MAX_TV + t;
#pragma unroll
        for (int dt = 0; dt < 6; dt++)
          st_b64(ws, (uint32_t)(L.cattp + (prow * HD + 16 * dt + 4 * g4) * 2),
                 u32x2{pack_bf16x2(o[dt][0], o[dt][1]), pack_bf16x2(o[dt][2], o[dt][3])});
        if (g4 == 0) st_b64(ws, (uint32_t)(L.cml + prow * 8), u32x2{as_u32(mx), as_u32(ps)});
      }
    }
  }
}

// attn[b Tv + t][96 h + d] = sum_c w_c O_c. A row's 96 dims on 12 lanes of 8 dims, five rows per wave
// (lanes 60-63 idle), so batch 16's 3840 rows take one trip of the 256 x 4 waves (3.34 -> 2.06 us per
// layer against two trips of 24 lanes x 4 dims). Like the norms, rows go wave-major over blockIdx, so
// consecutive rows land on different XCDs and a short stage uses all eight (norm-major over the
// XCD-major index left four XCDs idle at 480 rows: 34.54 -> 34.29 ms per launch).
__device__ __forceinline__ void stage_comb(const Params& p, rsrc_t ws) {
  const Layout& L = p.L;
  const int lane = lane_id(), sub = lane / 12;
  const int d0 = lane < 60 ? 8 * (lane - 12 * sub) : 0;
  const int nkc = (p.Lk + KCH - 1) / KCH;
  const int rows = p.B * NH * p.Tv;
#pragma unroll 1
  for (int R0 = (wave_id() * NWG + (int)blockIdx.x) * 5; R0 < rows; R0 += NWG * NWAVE * 5) {
    const int R = R0 + sub;
    const bool valid = R < rows && lane < 60;
    const int Rc = valid ? R : R0;
    const int t = Rc % p.Tv, bh = Rc / p.Tv, h = bh % NH, b = bh / NH;
    const size_t row0 = ((size_t)bh * L.NKC) * MAX_TV + t;
    float Mx = -1e30f, den = 0.f;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
    for (int c0 = 0; c0 < nkc; c0 += 8) {
      u32x2 ml[8];
      u32x4 v[8];
#pragma unroll
      for (int c = 0; c < 8; c++) {
        const size_t prow = row0 + (size_t)(c0 + c < nkc ? c0 + c : c0) * MAX_TV;
        ml[c] = ldb64<kCpSc1>(ws, (uint32_t)(L.cml + prow * 8));
        v[c] = ldb128<kCpSc1>(ws, (uint32_t)(L.cattp + (prow * HD + d0) * 2));
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
        for (int i = 0; i < 4; i++) {
          acc[2 * i] = acc[2 * i] * sa + sc * bf_lo(v[c][i]);
          acc[2 * i + 1] = acc[2 * i + 1] * sa + sc * bf_hi(v[c][i]);
        }
      }
    }
    if (valid) {
      const float inv = 1.0f / den;
      st_b128(ws, (uint32_t)L.attn + afrag(b * p.Tv + t, HD * h + d0, D),
              u32x4{pack_bf16x2(acc[0] * inv, acc[1] * inv), pack_bf16x2(acc[2] * inv, acc[3] * inv),
                    pack_bf16x2(acc[4] * inv, acc[5] * inv), pack_bf16x2(acc[6] * inv, acc[7] * inv)});
    }
  }
}

// ---------------------------------------------------------------- the kernel
constexpr uint32_t RING_BYTES = 147 * 1024;      // GEMM ring / attention tiles
constexpr uint32_t LDS_BYTES = RING_BYTES + 256;  // + the split-K fixup flag

__device__ __forceinline__ void mark(const Params& p, int idx, uint64_t& t0) {
  if (p.stage_cycles && blockIdx.x == 0 && threadIdx.x == 0) {
    const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
    p.stage_cycles[idx] += t1 - t0;
    t0 = t1;
  }
}

// (32 WM) x (32 WN) tiles for every GEMM but gate/up, (32 WM) x (32 WNG) for gate/up.
template <int WM, int WN, int WNG>
__global__ void __launch_bounds__(NTHR, 1) ma2_kernel(Params p) {
  static_assert(GemmShape<WM, WN>::LDS <= RING_BYTES && GemmShape<WM, WNG>::LDS <= RING_BYTES, "LDS budget");
  const Layout& L = p.L;
  const rsrc_t ws = rsrc_all(p.ws);
  const rsrc_t xtr = make_rsrc(p.x_t, (uint32_t)((size_t)p.B * p.xt_rows * AD * 4));
  Grid grid;
  grid.flags = reinterpret_cast<uint64_t*>(p.ws + OFF_FLAGS);
  grid.err = reinterpret_cast<unsigned*>(p.ws + OFF_CTRL + 8);
  const uint64_t seq = ld_flag(reinterpret_cast<const uint64_t*>(p.ws + OFF_CTRL));
  grid.e = seq << 32;
  if (threadIdx.x == 0 && xcc_id() != (blockIdx.x & 7u)) atomicOr(grid.err, kErrXcd);
  if (blockIdx.x == 0 && threadIdx.x == 0)
    __hip_atomic_store(reinterpret_cast<unsigned*>(p.ws + kWsOwner), kOwnerMa2Generic, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  const int NL = p.NL;
  const float dt = 1.0f / (float)p.S;
  uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  GemmArgs gx{reinterpret_cast<const bf16*>(p.ws + L.xn), nullptr, D, D, L.M};
  GemmArgs ga{reinterpret_cast<const bf16*>(p.ws + L.attn), nullptr, D, D, L.M};
  GemmArgs gh{reinterpret_cast<const bf16*>(p.ws + L.h), nullptr, FF, FF, L.M};
  auto sync = [&](int idx) {
    mark(p, idx, t0);
    grid_sync(grid);
    mark(p, 15, t0);
  };
  // Small tiles (FIX): the last K-split of each tile sums the partials and applies the bias (and
  // the gate/up activation); large tiles: the consumer stage sums the partials (and a GATE stage
  // applies the activation), which spreads the reduction over all workgroups.
  constexpr bool FIX = WM == 1;
  unsigned* cnt = reinterpret_cast<unsigned*>(p.ws + L.cnt);
  // xn and attn are fragment-ordered (AF); h stays row-major, written whole rows at a time by the
  // gate/up epilogue (as fragments, 4 bytes per lane into 16-byte slots, GU took 14.2 instead of
  // 11.3 µs per layer at batch 16)
  auto gemm = [&](auto af, GemmArgs& g, const bf16* W, int N, int K, int ks, uint32_t part, uint32_t yfin,
                  const float* bias) {
    constexpr bool AF = decltype(af)::value;
    g.W = W;
    if constexpr (FIX) {
      FinBias f{ws, yfin, N, bias};
      gemm_stage_fixup<WM, WN, AF>(g, N, K, ks, ws, part, L.MP, cnt, RING_BYTES, f);
    } else {
      EpiPartN e{{}, ws, part, L.MP, N, 0};
      // a three-step ring where it fits (the 128 x 64 tiles of batch 16: QKV 8.15 -> 7.32 us per layer,
      // 35.47 -> 34.95 ms per launch)
      constexpr int RD = 3 * GemmShape<WM, WN, AF>::STEP <= RING_BYTES ? 3 : 2;
      gemm_stage<WM, WN, AF, RD, true>(g, N, K, ks, e);
    }
  };
  const std::true_type frag;
  const std::false_type rows;
#pragma unroll 1
  for (int step = 0; step < p.S; step++) {
#pragma unroll 1
    for (int l = 0; l < NL; l++) {
      const float* mo = p.mods + ((size_t)step * NL + l) * 9 * D;  // [3 norms][scale, shift, gate][D]
      const YSrc ydn{L.yo, L.part, L.ks_dn, D, p.b_dn + (size_t)(l > 0 ? l - 1 : 0) * D};
      const YSrc yso{L.yo, L.part, L.ks_d, D, p.b_so + (size_t)l * D};
      const YSrc yco{L.yo, L.part, L.ks_d, D, p.b_co + (size_t)l * D};
      const YSrc yqkv{L.yqkv, L.pqkv, L.ks_qkv, QKVN, p.b_qkv + (size_t)l * QKVN};
      const YSrc ycq{L.yq, L.pq, L.ks_d, D, p.b_cq + (size_t)l * D};
      if (l == 0)
        stage_norm<0, FIX>(p, ws, xtr, ydn, nullptr, mo, mo + D, 0.f);
      else
        stage_norm<1, FIX>(p, ws, xtr, ydn, mo - 9 * D + 8 * D, mo, mo + D, 0.f);  // gate: mlp of layer l-1
      sync(0);
      gemm(frag, gx, p.w_qkv + (size_t)l * QKVN * D, QKVN, D, L.ks_qkv, (uint32_t)L.pqkv, (uint32_t)L.yqkv, yqkv.bias);
      sync(1);
      stage_satt<FIX>(p, ws, yqkv);
      sync(2);
      gemm(frag, ga, p.w_so + (size_t)l * D * D, D, D, L.ks_d, (uint32_t)L.part, (uint32_t)L.yo, yso.bias);
      sync(3);
      stage_norm<1, FIX>(p, ws, xtr, yso, mo + 2 * D, mo + 3 * D, mo + 4 * D, 0.f);
      sync(4);
      gemm(frag, gx, p.w_cq + (size_t)l * D * D, D, D, L.ks_d, (uint32_t)L.pq, (uint32_t)L.yq, ycq.bias);
      mark(p, 5, t0);
      grid_sync(grid, [&] { catt_prefetch(p, l); });
      mark(p, 15, t0);
      stage_catt<FIX>(p, ws, l, ycq, true);
      sync(6);
      stage_comb(p, ws);
      sync(7);
      gemm(frag, ga, p.w_co + (size_t)l * D * D, D, D, L.ks_d, (uint32_t)L.part, (uint32_t)L.yo, yco.bias);
      sync(8);
      stage_norm<1, FIX>(p, ws, xtr, yco, mo + 5 * D, mo + 6 * D, mo + 7 * D, 0.f);
      sync(9);
      gx.W = p.w_gu + (size_t)l * GUN * D;
      if constexpr (FIX) {
        FinSiluGate f{ws, (uint32_t)L.h, p.b_gu + (size_t)l * GUN};
        gemm_stage_fixup<WM, WNG, true>(gx, GUN, D, L.ks_gu, ws, (uint32_t)L.pgu, L.MP, cnt, RING_BYTES, f);
      } else if (L.ks_gu == 1) {  // one pass of tiles covers the grid: gate fused into the epilogue
        EpiSiluGate e{ws, (uint32_t)L.h, p.b_gu + (size_t)l * GUN, 0};
        gemm_stage<WM, WNG, true, 2, true>(gx, GUN, D, 1, e);
        mark(p, 10, t0);
      } else {
        EpiPartN e{{}, ws, (uint32_t)L.pgu, L.MP, GUN, 0};
        gemm_stage<WM, WNG, true, 2, true>(gx, GUN, D, L.ks_gu, e);
        sync(10);
        stage_gate(p, ws, l);
      }
      sync(11);
      gemm(rows, gh, p.w_dn + (size_t)l * D * FF, D, FF, L.ks_dn, (uint32_t)L.part, (uint32_t)L.yo,
           p.b_dn + (size_t)l * D);
      sync(12);
    }
    const float* ml = p.mods + ((size_t)step * NL + NL - 1) * 9 * D;
    const float* mf = p.mod_final + (size_t)step * 2 * D;
    const YSrc ydn{L.yo, L.part, L.ks_dn, D, p.b_dn + (size_t)(NL - 1) * D};
    stage_norm<2, FIX>(p, ws, xtr, ydn, ml + 8 * D, mf, mf + D, dt);
    sync(13);
  }
  if (blockIdx.x == 0 && threadIdx.x == 0)
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p.ws + OFF_CTRL), seq + 1, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Tile shapes: batches of up to 64 tokens use 32-token x 64-row tiles; larger ones 96 x 64 tiles,
// except gate/up on 96 x 128. At batch 16 (480 tokens = 5 x 96, no padded rows) the 96-token tiles
// keep every stage within one pass of the 256 workgroups (QKV 180 tiles without a K split, the
// 768 x 768 projections split 3, down 4, gate/up 240 tiles) and copy 24 activation fragments per
// k-step where two 64-row groups took 32: 33.43 -> 31.73 ms per launch against 128-token tiles
// (QKV 7.0 -> 5.8, gate/up 11.0 -> 9.7 us per layer), which had taken 38.3 -> 36.1 ms against 128 x 128
// everywhere.
constexpr int SMALL_M = 64;
__host__ inline bool small_cfg(int M) { return M <= SMALL_M; }
__host__ inline Layout layout_for(int B, int Tv, int Lkmax) {
  return small_cfg(B * Tv) ? layout(B, Tv, Lkmax, 32, 64, 64) : layout(B, Tv, Lkmax, 96, 64, 128);
}

}  // namespace ma2
}  // namespace fa

// ================================================================= host C ABI
using namespace fa;

extern "C" size_t fa_ma2_workspace_bytes(int batch, int Tv, int Lkmax) {
  if (batch < 1 || Tv < 1 || Tv > ma2::MAX_TV || Lkmax < 16 || (size_t)batch * Tv > (size_t)ma2::MAX_TOKENS) return 0;
  if (ma2_bs1_eligible(batch, Tv, Lkmax)) return ma2_bs1_workspace_bytes();
  const size_t n = ma2::layout_for(batch, Tv, Lkmax).total;
  return n < 0xffffffffull ? n : 0;
}

extern "C" int fa_ma2_max_batch(void) { return ma2::MAX_TOKENS / ma2::MAX_TV; }

extern "C" int fa_ma2_workspace_init(void* workspace, size_t bytes, fa_stream_t stream) {
  return fa_pi05_workspace_init(workspace, bytes, stream);
}

extern "C" int fa_ma2_read_status(const void* workspace, unsigned* status) {
  return fa_pi05_read_status(workspace, status);
}

extern "C" int fa_ma2_flow(const fa_ma2_args* a, fa_stream_t stream) {
  using namespace fa::ma2;
  if (!a) return host::fail(FA_ERR_INVALID_ARG, "fa_ma2_flow: args is NULL");
  if (a->weight_dtype != FA_DTYPE_BF16)
    return host::fail(FA_ERR_UNSUPPORTED, "fa_ma2_flow: only bf16 weights are implemented (weight_dtype=%d)",
                      a->weight_dtype);
  const void* ptrs[] = {a->w_qkv, a->w_so, a->w_cq, a->w_co, a->w_gu, a->w_dn, a->b_qkv, a->b_so, a->b_cq,
                        a->b_co, a->b_gu, a->b_dn, a->mods, a->mod_final, a->rope_cos, a->rope_sin, a->w_ain,
                        a->b_ain, a->w_aout, a->b_aout, a->kctx, a->vtctx, a->x_t, a->workspace};
  const char* names[] = {"w_qkv", "w_so", "w_cq", "w_co", "w_gu", "w_dn", "b_qkv", "b_so", "b_cq", "b_co",
                         "b_gu", "b_dn", "mods", "mod_final", "rope_cos", "rope_sin", "w_ain", "b_ain",
                         "w_aout", "b_aout", "kctx", "vtctx", "x_t", "workspace"};
  for (int i = 0; i < 24; i++) {
    if (!ptrs[i]) return host::fail(FA_ERR_INVALID_ARG, "fa_ma2_flow: %s is NULL", names[i]);
    if (reinterpret_cast<uintptr_t>(ptrs[i]) & 15)
      return host::fail(FA_ERR_INVALID_ARG, "fa_ma2_flow: %s is not 16-byte aligned", names[i]);
  }
  if (reinterpret_cast<uintptr_t>(a->workspace) & 255)
    return host::fail(FA_ERR_INVALID_ARG, "fa_ma2_flow: workspace is not 256-byte aligned");
  if (a->num_layers < 1 || a->num_steps < 1 || a->Tv < 1 || a->Tv > MAX_TV || a->Lk < 1 || a->adim < 0 ||
      a->adim > AD || a->batch < 1)
    return host::fail(FA_ERR_INVALID_ARG, "fa_ma2_flow: need num_layers>=1, num_steps>=1, 1<=Tv<=%d, Lk>=1, "
                      "0<=adim<=32, batch>=1 (got NL=%d S=%d Tv=%d Lk=%d adim=%d batch=%d)", MAX_TV, a->num_layers,
                      a->num_steps, a->Tv, a->Lk, a->adim, a->batch);
  if (a->Lkmax < a->Lk || (a->Lkmax & 15))
    return host::fail(FA_ERR_INVALID_ARG, "fa_ma2_flow: Lkmax=%d must be a multiple of 16 and >= Lk=%d", a->Lkmax,
                      a->Lk);
  if (a->xt_rows < a->Tv)
    return host::fail(FA_ERR_INVALID_ARG, "fa_ma2_flow: xt_rows=%d < Tv=%d", a->xt_rows, a->Tv);
  if ((size_t)a->batch * a->Tv > (size_t)MAX_TOKENS)
    return host::fail(FA_ERR_INVALID_ARG, "fa_ma2_flow: batch x Tv = %d exceeds %d tokens", a->batch * a->Tv,
                      MAX_TOKENS);
  if ((size_t)a->batch * a->num_layers * a->Lkmax * D * 2 >= 0xffffffffull)
    return host::fail(FA_ERR_INVALID_ARG, "fa_ma2_flow: context caches exceed the 4 GB buffer range");
  const size_t need = fa_ma2_workspace_bytes(a->batch, a->Tv, a->Lkmax);
  if (need == 0 || a->workspace_bytes < need)
    return host::fail(FA_ERR_INVALID_ARG, "fa_ma2_flow: workspace_bytes=%zu < required %zu", a->workspace_bytes,
                      need);
  if (ma2_bs1_eligible(a->batch, a->Tv, a->Lkmax)) return ma2_bs1_launch(a, stream);
  const bool sm = small_cfg(a->batch * a->Tv);
  const void* kern = sm ? (const void*)ma2_kernel<1, 2, 2> : (const void*)ma2_kernel<3, 2, 4>;
  int rc = host::check_device(kern, NTHR, LDS_BYTES, NWG, "fa_ma2_flow");
  if (rc != FA_OK) return rc;
  Params p;
  p.w_qkv = static_cast<const bf16*>(a->w_qkv);
  p.w_so = static_cast<const bf16*>(a->w_so);
  p.w_cq = static_cast<const bf16*>(a->w_cq);
  p.w_co = static_cast<const bf16*>(a->w_co);
  p.w_gu = static_cast<const bf16*>(a->w_gu);
  p.w_dn = static_cast<const bf16*>(a->w_dn);
  p.b_qkv = a->b_qkv;
  p.b_so = a->b_so;
  p.b_cq = a->b_cq;
  p.b_co = a->b_co;
  p.b_gu = a->b_gu;
  p.b_dn = a->b_dn;
  p.mods = a->mods;
  p.mod_final = a->mod_final;
  p.rope_cos = a->rope_cos;
  p.rope_sin = a->rope_sin;
  p.w_ain = a->w_ain;
  p.b_ain = a->b_ain;
  p.w_aout = static_cast<const bf16*>(a->w_aout);
  p.b_aout = a->b_aout;
  p.kctx = static_cast<const bf16*>(a->kctx);
  p.vtctx = static_cast<const bf16*>(a->vtctx);
  p.x_t = a->x_t;
  p.stage_cycles = a->stage_cycles;
  p.ws = static_cast<unsigned char*>(a->workspace);
  p.L = layout_for(a->batch, a->Tv, a->Lkmax);
  if (sm && (uint32_t)p.L.ntiles > kWsMaxCounters)
    return host::fail(FA_ERR_UNSUPPORTED, "fa_ma2_flow: %d fixup tiles exceed %u counters", p.L.ntiles, kWsMaxCounters);
  p.NL = a->num_layers;
  p.Lk = a->Lk;
  p.Lkmax = a->Lkmax;
  p.Tv = a->Tv;
  p.adim = a->adim;
  p.S = a->num_steps;
  p.B = a->batch;
  p.xt_rows = a->xt_rows;
  void* args[] = {&p};
  return host::coop_launch(kern, NWG, NTHR, args, LDS_BYTES, stream, "fa_ma2_flow");
}
