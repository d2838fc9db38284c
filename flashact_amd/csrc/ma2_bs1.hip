// MolmoAct2 flow loop at batch 1 (the MolmoAct2 workload: Tv = 30 action tokens, Lk = 493 context
// keys): the latency-bound case, laid out on the XCDs like the pi0.5 batch-1 kernel.
//
// One cooperative launch of 256 workgroups x 4 waves. XCD g = blockIdx % 8 owns attention head g;
// rank r = blockIdx / 8 (0..31) owns token r in the norm stages. Per layer ([X] = XCD barrier,
// {E} = cross-XCD exchange of fp32 partial sums, the only data that leaves an XCD):
//   N_msa  token r: x += g_mlp * (sum of the 8 down partials + b_dn) (x lives in LDS), adaRMS -> xn
//          (every XCD keeps its own identical copy of x and xn)                                [X]
//   QKV    ranks 0..17: 16 of the head's 288 q/k/v rows x 768, + b_qkv                          [X]
//   SATT   rank 0: per-head RMS of q and k, RoPE, softmax(q k^T / sqrt(96)) v over the tokens  [X]
//   SO     all ranks: 24 rows of W_so[:, 96g..96g+96) x attn_g -> partial                      {E}
//   N_mca  as N_msa with g_msa, b_so                                                            [X]
//   CQ     ranks 0..5: 16 of the head's 96 q rows x 768, + b_cq                                  [X]
//   CATT   ranks 0..15: context keys 32r..32r+31 of head g -> normalised partial O + (m, l)    [X]
//   COMB   token r: combine the key chunks -> attn_g                                            [X]
//   CO     as SO with W_co                                                                      {E}
//   N_mlp  as N_msa with g_mca, b_co                                                            [X]
//   GU     all ranks: 24 interleaved gate/up rows of the head's slice f in [384g, 384g+384)
//          -> h = silu(g + b_g) (u + b_u)                                                       [X]
//   DN     all ranks: 24 rows of W_dn[:, 384g..384g+384) x h_g -> partial                      {E}
// (the reference runs every stage behind a grid-wide barrier: src/molmoact2/mk_ma2.cu:286-561).
// Weight fragments of the next GEMM stage (and the context K/V of the attention stage) are loaded
// into registers before each wait, so HBM latency overlaps the synchronisation.
// GEMMs: v_mfma_f32_16x16x32_bf16 with 16 weight rows as A and 16 tokens as B; activations are
// kept in MFMA fragment order in each XCD's L2 (plain stores, sc1 loads).
#include "engine.h"
#include "ma2_attn.h"
#include "../../include/flashact_mi355x.h"
#include "fa_host.h"

namespace fa {
namespace ma2x {
using namespace fa::eng;
using namespace fa::ma2att;

constexpr int D = 768, FF = 3072, AD = 32, QKVN = 3 * D, GUN = 2 * FF;
constexpr int NX = 8, NR = 32;
constexpr int TP = 32;   // token slots (Tv <= 32)
constexpr int KPR = 32;  // context keys per cross-attention rank (Lk <= 512)
constexpr int MAX_LK = NR / 2 * KPR;

// ---- workspace (bytes)
constexpr uint32_t OFF_CTRL = 0;     // u64 seq, u32 err @8, u32 exchange parity bases @12, @16
constexpr uint32_t OFF_XFLAG = 1024; // [8 XCD][32 rank][4 wave] u64 epochs
constexpr uint32_t OFF_XP = kWsDataBase;  // [2 buffers][8 XCD][32 tokens][768] f32 (parity-tagged)
constexpr uint32_t XP_BYTES = 2 * NX * TP * D * 4;
// per-XCD block (stride XB): activations in MFMA fragment order and small fp32 intermediates.
// X_QKV and X_QC are lane-major, in the order the attention stages read them: 16-byte group
// (token tile tt, slot s, lane lr + 16 g4) holds dims 16 (s % 6) + 4 g4 .. + 3 of part s / 6
// (q | k | v) of token 16 tt + lr, so each of those loads reads 1 KB contiguous, and the RoPE
// partners j, j + 48 sit in slots s, s + 3 of one lane.
constexpr uint32_t X_XN = 0;                          // [32][768] bf16 fragments
constexpr uint32_t X_QKV = X_XN + TP * D * 2;         // [2][18][64] f32x4 (q | k | v of head g, + bias)
constexpr uint32_t X_ATT = X_QKV + TP * 288 * 4;      // [32][96] bf16 fragments
constexpr uint32_t X_QC = X_ATT + TP * HD * 2;        // [2][6][64] f32x4 (+ bias)
constexpr uint32_t X_CP = X_QC + TP * HD * 4;         // [16 chunks][32][96] bf16 partials
constexpr uint32_t X_CML = X_CP + 16 * TP * HD * 2;   // [16][32] (m, l) f32
constexpr uint32_t X_H = X_CML + 16 * TP * 8;         // [32][384] bf16 fragments
constexpr uint32_t XB = (X_H + TP * 384 * 2 + 4095) / 4096 * 4096;
constexpr uint32_t OFF_XCD = OFF_XP + XP_BYTES;
constexpr uint32_t WS_BYTES = OFF_XCD + NX * XB;
static_assert(OFF_XFLAG + NX * NR * 4 * 8 <= kWsCounters, "flags stay below the fixup counters");

// ---- LDS
constexpr uint32_t L_ATT = 0;                       // attention fragments (36 KB)
constexpr uint32_t L_RED = 36 * 1024;               // cross-wave reduction [4 waves][4][64] f32x4 (16 KB)
constexpr uint32_t L_X = L_RED + 16 * 1024;         // residual x of token r [768] f32
constexpr uint32_t L_XT = L_X + D * 4;              // x_t of token r [32] f32
constexpr uint32_t L_MISC = L_XT + AD * 4;          // [4 waves][768] f32 exchange partial sums
constexpr uint32_t L_ROPE = L_MISC + 4 * D * 4;     // rank 0: RoPE cos | sin [2][32 tokens][48] f32
constexpr uint32_t LDS_BYTES = L_ROPE + 2 * TP * 48 * 4;

struct Params {
  const bf16 *w_qkv, *w_so, *w_cq, *w_co, *w_gu, *w_dn;
  const float *b_qkv, *b_so, *b_cq, *b_co, *b_gu, *b_dn;
  const float *mods, *mod_final, *rope_cos, *rope_sin, *w_ain, *b_ain;
  const bf16* w_aout;
  const float* b_aout;
  const bf16* kctx;   // [NL][Lkmax][768]
  const bf16* vtctx;  // [NL][768][Lkmax]
  float* x_t;         // [xt_rows][32]
  unsigned long long* stage_cycles;
  unsigned char* ws;
  int NL, Lk, Lkmax, Tv, adim, S;
};

struct Ctx {
  int g, r, w, lane, lr, lq;
  rsrc_t ws;
  uint32_t xb;       // byte offset of this XCD's block
  uint64_t* xflag;   // this XCD's 32 rank flags
  unsigned* err;
  uint64_t e;
};

__device__ __forceinline__ uint32_t afo(int KS, int m, int k) {  // fragment-order byte offset
  return (uint32_t)((((m >> 4) * KS + (k >> 5)) * 64 + (m & 15) + 16 * ((k & 31) >> 3)) * 16 + (k & 7) * 2);
}
__device__ __forceinline__ u32x4 wfrag(const bf16* W, int ldw, int row, int k, int lq) {
  return *reinterpret_cast<const u32x4*>(W + (size_t)row * ldw + k + 8 * lq);
}
__device__ __forceinline__ u32x4 tag(f32x4 v, unsigned par) {
  u32x4 u = as_u32x4(v);
#pragma unroll
  for (int i = 0; i < 4; i++) u[i] = (u[i] & ~1u) | par;
  return u;
}
__device__ __forceinline__ unsigned mism(u32x4 v, unsigned par) {
  return ((v[0] ^ par) | (v[1] ^ par) | (v[2] ^ par) | (v[3] ^ par)) & 1u;
}
__device__ __forceinline__ bool aborted(const Ctx& c) {
  return __hip_atomic_load(c.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & kErrSpin;
}

// ---- XCD barrier on per-wave epoch flags [XCD][rank][wave]. Work that does not depend on the
// barrier (weight prefetch) goes between arrive and wait. The flags are plain stores, which stay in
// the XCD's L2 where the other ranks' sc1 polls find them (a device-scope store went out to memory
// and back: 15.8 -> 13.0 ms per chunk with the plain store); only this XCD reads them, and the
// prologue's grid-wide barrier, read across XCDs, stores them device-scope. Every wave publishes its
// own arrival and polls the XCD's 128 flags itself (one 16-byte sc1 load per lane), with no
// workgroup barrier. A wave passes only after every wave of the XCD, its own
// workgroup's included, has drained its global and LDS operations and published, so LDS written or
// read before the barrier by a sibling wave is settled for all of them. Against one flag per
// workgroup (a workgroup barrier, then wave 0 polling 32 flags while the others wait at a second
// workgroup barrier): 11.48-11.55 -> 11.15-11.17 ms per chunk.
__device__ __forceinline__ void xarrive(Ctx& c) {
  __builtin_amdgcn_s_waitcnt(0);  // this wave's global and LDS operations are complete
  c.e += 1;
  if (c.lane == 0) __hip_atomic_store(c.xflag + c.r * 4 + c.w, c.e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void xwait(Ctx& c) {
  if (!aborted(c)) {
    const rsrc_t fr = make_rsrc(c.xflag, NR * 4 * 8);
    for (unsigned it = 0;; ++it) {
      const u32x4 v = ldb128<kCpSc1>(fr, (uint32_t)c.lane * 16);
      const uint64_t f0 = ((uint64_t)v[1] << 32) | v[0], f1 = ((uint64_t)v[3] << 32) | v[2];
      if (__builtin_amdgcn_ballot_w64(f0 < c.e || f1 < c.e) == 0) break;
      if (it > kSpinCap) {
        if (c.lane == 0) atomicOr(c.err, kErrSpin);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  asm volatile("" ::: "memory");
}

// ---- exchange: the 8 XCD partials of token t (fp32, lowest mantissa bit = parity) -------------
// Wave w reads XCDs 2w, 2w+1 (columns 4 lane + 256 k, k < 3): polls a hint word per XCD with a
// sleep, loads everything, re-reads groups whose parity is stale; the pair sum goes to LDS and
// wave 0 adds the 4 pair sums in a fixed order (every XCD computes the same x).
__device__ __forceinline__ void xread_token(const Ctx& c, int buf, int t, unsigned par, f32x4 (&sum)[3]) {
  const uint32_t b0 = OFF_XP + (uint32_t)((((buf * NX + 2 * c.w) * TP + t) * D + 4 * c.lane) * 4);
  const uint32_t xs = (uint32_t)(TP * D * 4);  // next XCD
  if (!aborted(c)) {
    const uint32_t hint = OFF_XP + (uint32_t)((((buf * NX + 2 * c.w + (c.lane & 1)) * TP + t) * D + D - 4) * 4);
    for (unsigned it = 0;; ++it) {
      const u32x4 h = ldb128<kCpSc1>(c.ws, hint);
      if (__builtin_amdgcn_ballot_w64(c.lane < 2 && mism(h, par)) == 0) break;
      if ((it & 1023) == 1023 && (aborted(c) || it > kSpinCap)) break;
      __builtin_amdgcn_s_sleep(4);
    }
  }
  u32x4 v[2][3];
#pragma unroll
  for (int x = 0; x < 2; x++)
#pragma unroll
    for (int k = 0; k < 3; k++) v[x][k] = ldb128<kCpSc1>(c.ws, b0 + x * xs + 256 * k * 4);
  for (unsigned it = 0;; ++it) {
    unsigned bad = 0;
#pragma unroll
    for (int x = 0; x < 2; x++)
#pragma unroll
      for (int k = 0; k < 3; k++) bad |= mism(v[x][k], par) << (x * 3 + k);
    if (__builtin_amdgcn_ballot_w64(bad != 0) == 0) break;
    if ((it & 255) == 255 && (aborted(c) || it > kSpinCap)) {
      if (c.lane == 0) atomicOr(c.err, kErrSpin);
      break;
    }
    __builtin_amdgcn_s_sleep(4);
#pragma unroll
    for (int x = 0; x < 2; x++)
#pragma unroll
      for (int k = 0; k < 3; k++)
        if ((bad >> (x * 3 + k)) & 1u) v[x][k] = ldb128<kCpSc1>(c.ws, b0 + x * xs + 256 * k * 4);
  }
  float* part = reinterpret_cast<float*>(lds + L_MISC) + c.w * D;
#pragma unroll
  for (int k = 0; k < 3; k++)
    *reinterpret_cast<f32x4*>(part + 4 * c.lane + 256 * k) = as_f32x4(v[0][k]) + as_f32x4(v[1][k]);
  __syncthreads();
  const float* p0 = reinterpret_cast<const float*>(lds + L_MISC);
#pragma unroll
  for (int k = 0; k < 3; k++) {
    const int d = 4 * c.lane + 256 * k;
    sum[k] = (*reinterpret_cast<const f32x4*>(p0 + d) + *reinterpret_cast<const f32x4*>(p0 + D + d)) +
             (*reinterpret_cast<const f32x4*>(p0 + 2 * D + d) + *reinterpret_cast<const f32x4*>(p0 + 3 * D + d));
  }
}

// ---- norm stages (token t = rank r, wave 0 after the exchange read) ---------------------------
// MODE 0: x = embed(x_t); MODE 1: x += gate * (sum + bias); MODE 2: as 1, then the final norm,
// the action projection and x_t[:, :adim] += dt * v.
template <int MODE>
__device__ __forceinline__ void stage_norm(const Params& p, const Ctx& c, int buf, unsigned par, const float* bias,
                                           const float* gate, const float* scale, const float* shift, float dt) {
  const int t = c.r;
  if (t >= p.Tv) return;
  f32x4 sum[3];
  if (MODE != 0) xread_token(c, buf, t, par, sum);
  if (c.w != 0) return;
  float* xres = reinterpret_cast<float*>(lds + L_X);
  float* xt = reinterpret_cast<float*>(lds + L_XT);
  f32x4 x[3];
  if (MODE == 0) {
    float xa[AD];
#pragma unroll
    for (int a = 0; a < AD; a++) xa[a] = xt[a];
#pragma unroll
    for (int k = 0; k < 3; k++) {
      const int d = 4 * c.lane + 256 * k;
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
#pragma unroll
    for (int k = 0; k < 3; k++) {
      const int d = 4 * c.lane + 256 * k;
      x[k] = *reinterpret_cast<const f32x4*>(xres + d) +
             *reinterpret_cast<const f32x4*>(gate + d) * (sum[k] + *reinterpret_cast<const f32x4*>(bias + d));
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < 3; k++) ss += x[k][0] * x[k][0] + x[k][1] * x[k][1] + x[k][2] * x[k][2] + x[k][3] * x[k][3];
  const float rr = rsqrtf(wave_sum(ss) / (float)D + 1e-6f);
  f32x4 h[3];
#pragma unroll
  for (int k = 0; k < 3; k++) {
    const int d = 4 * c.lane + 256 * k;
    const f32x4 sc = *reinterpret_cast<const f32x4*>(scale + d);
    const f32x4 sh = *reinterpret_cast<const f32x4*>(shift + d);
#pragma unroll
    for (int i = 0; i < 4; i++) h[k][i] = x[k][i] * rr * (1.0f + sc[i]) + sh[i];
  }
  if (MODE != 2) {
#pragma unroll
    for (int k = 0; k < 3; k++) {
      const int d = 4 * c.lane + 256 * k;
      *reinterpret_cast<f32x4*>(xres + d) = x[k];
      *reinterpret_cast<u32x2*>(p.ws + c.xb + X_XN + afo(D / 32, t, d)) =
          u32x2{pack_bf16x2(h[k][0], h[k][1]), pack_bf16x2(h[k][2], h[k][3])};
    }
  } else {
    float acc = 0.f;  // lane a < adim ends with v[a]
#pragma unroll 1
    for (int a = 0; a < p.adim; a++) {
      float s = 0.f;
#pragma unroll
      for (int k = 0; k < 3; k++) {
        const u32x2 wv = *reinterpret_cast<const u32x2*>(p.w_aout + (size_t)a * D + 4 * c.lane + 256 * k);
        s += bf_lo(wv[0]) * h[k][0] + bf_hi(wv[0]) * h[k][1] + bf_lo(wv[1]) * h[k][2] + bf_hi(wv[1]) * h[k][3];
      }
      s = wave_sum(s);
      if (c.lane == a) acc = s;
    }
    if (c.lane < p.adim) xt[c.lane] += dt * (acc + p.b_aout[c.lane]);
  }
}

// ---- GEMM pieces -------------------------------------------------------------------------------
// One 16-row weight tile over all 32 tokens, K = 768 split over the 4 waves (k-steps 6w..6w+5;
// wf = this wave's weight fragments, loaded ahead). The four partial sums meet in LDS; waves 0/1
// finish token tiles 0/1: + bias, columns col0 + 4 lq .. + 3 (of ns 96-column parts) into the
// lane-major layout of X_QKV / X_QC at `out` (each store instruction writes 4 runs of 256 bytes;
// row-major [token][column] rows read back by lanes 96 bytes apart took the self attention's loads
// through about seven 128-byte lines per kilobyte used).
__device__ __forceinline__ void gemm16(const Params& p, const Ctx& c, const u32x4 (&wf)[6], uint32_t out, int ns,
                                       int col0, const float* bias) {
  f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  u32x4 b[2][6];
#pragma unroll
  for (int j = 0; j < 6; j++)
#pragma unroll
    for (int tt = 0; tt < 2; tt++)
      b[tt][j] = ldb128<kCpSc1>(c.ws, c.xb + X_XN + (uint32_t)(((tt * (D / 32) + 6 * c.w + j) * 64 + c.lane) * 16));
#pragma unroll
  for (int j = 0; j < 6; j++)
#pragma unroll
    for (int tt = 0; tt < 2; tt++) acc[tt] = mfma16(wf[j], b[tt][j], acc[tt]);
  f32x4* red = reinterpret_cast<f32x4*>(lds + L_RED);
#pragma unroll
  for (int tt = 0; tt < 2; tt++) red[(c.w * 2 + tt) * 64 + c.lane] = acc[tt];
  __syncthreads();
  if (c.w < 2) {
    const int tt = c.w;
    f32x4 s = (red[(0 * 2 + tt) * 64 + c.lane] + red[(1 * 2 + tt) * 64 + c.lane]) +
              (red[(2 * 2 + tt) * 64 + c.lane] + red[(3 * 2 + tt) * 64 + c.lane]);
    s += *reinterpret_cast<const f32x4*>(bias + 4 * c.lq);
    const int col = col0 + 4 * c.lq, j = (col % HD) >> 2;  // 4-column group j of part col / 96
    const int slot = 6 * (col / HD) + (j >> 2);
    *reinterpret_cast<f32x4*>(p.ws + c.xb + out + (((tt * 6 * ns + slot) * 64 + c.lr + 16 * (j & 3)) * 16)) = s;
  }
}

// Weight row of the lane in a 24-row slice (two 16-row tiles; tile 1 uses rows 16..23, its lanes
// 8..15 load a row the slice does use and their results are dropped).
__device__ __forceinline__ int row24(int base, int rt, int lr) { return base + 16 * rt + ((rt == 1 && lr >= 8) ? lr - 8 : lr); }

// Partial-sum projection of this XCD's K-window onto 24 output rows (SO / CO: K = 96 over the
// head's attention output; DN: K = 384 over h). Wave w = (row tile w / 2, token tile w % 2); the
// tagged fp32 partial goes to exchange buffer `buf` with the parity bit `par`.
template <int NK>
__device__ __forceinline__ void proj24(const Params& p, const Ctx& c, const u32x4 (&wf)[NK], uint32_t act, int KS,
                                       int buf, unsigned par) {
  const int rt = c.w >> 1, tt = c.w & 1;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  u32x4 b[NK];
#pragma unroll
  for (int j = 0; j < NK; j++) b[j] = ldb128<kCpSc1>(c.ws, c.xb + act + (uint32_t)(((tt * KS + j) * 64 + c.lane) * 16));
#pragma unroll
  for (int j = 0; j < NK; j++) acc = mfma16(wf[j], b[j], acc);
  const int t = 16 * tt + c.lr;
  // Every token slot is written (zeros past Tv): a slot left over from an earlier launch with a
  // larger Tv could otherwise carry the parity this launch waits for.
  if (rt == 0 || c.lq < 2) {
    const int col = 24 * c.r + 16 * rt + 4 * c.lq;
    if (t >= p.Tv) acc = f32x4{0.f, 0.f, 0.f, 0.f};
    __builtin_amdgcn_raw_buffer_store_b128(tag(acc, par), c.ws,
                                           OFF_XP + (uint32_t)((((buf * NX + c.g) * TP + t) * D + col) * 4), 0,
                                           kCpSc1);
  }
}

// ---- self attention of head g (rank 0) --------------------------------------------------------
__device__ __forceinline__ void stage_satt(const Params& p, const Ctx& c) {
  const int tau = 16 * c.w + c.lr, g4 = c.lq;
  const bool tv = tau < p.Tv;
  float q[24], k[24], v[24];
  {
    // slots 0-5 / 6-11 / 12-17 of the lane: q / k / v, element 4 s + i = dim 16 s + 4 g4 + i (a wave
    // past Tv reads tile 0; lanes of tokens past Tv stay within their own four lanes and are
    // written as zeros below)
    const int tt = 16 * c.w < p.Tv ? c.w : 0;
    u32x4 r[18];
#pragma unroll
    for (int s = 0; s < 18; s++) r[s] = ldb128<kCpSc1>(c.ws, c.xb + X_QKV + (uint32_t)(((tt * 18 + s) * 64 + c.lane) * 16));
#pragma unroll
    for (int qq = 0; qq < 6; qq++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        q[4 * qq + i] = as_f32(r[qq][i]);
        k[4 * qq + i] = as_f32(r[6 + qq][i]);
        v[4 * qq + i] = as_f32(r[12 + qq][i]);
      }
  }
  rms96(q);
  rms96(k);
  // RoPE on split-half pairs (j, j + 48) = elements (4 s + i, 4 s + 12 + i) of the lane, s < 3
  const float* rope = reinterpret_cast<const float*>(lds + L_ROPE) + (tv ? tau : 0) * 48;  // staged by the prologue
#pragma unroll
  for (int s = 0; s < 3; s++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int j = 16 * s + 4 * g4 + i, a = 4 * s + i, b = a + 12;
      const float cs = rope[j], sn = rope[TP * 48 + j];
      const float q0 = q[a], q1 = q[b], k0 = k[a], k1 = k[b];
      q[a] = q0 * cs - q1 * sn;
      q[b] = q0 * sn + q1 * cs;
      k[a] = k0 * cs - k1 * sn;
      k[b] = k0 * sn + k1 * cs;
    }
  constexpr uint32_t SQ = 0, SK = 12 * 1024, SV = 24 * 1024;
  // q and k rows: each 4-dim group of the lane is half an 8-dim fragment slot (8-byte writes);
  // V^T is transposed, one element per write (pairing neighbouring tokens through DPP was slower)
  const uint32_t kr = kperm_row(tau);
  const unsigned keep = keep_mask(tv);
#pragma unroll
  for (int s = 0; s < 6; s++) {
    const int d = 16 * s + 4 * g4;
    const u32x2 qs = pack4(q, s, keep);
    const u32x2 ks = pack4(k, s, keep);
    *reinterpret_cast<u32x2*>(lds + L_ATT + SQ + ((tau >> 4) * 3 + (d >> 5)) * 1024 + frag_pos(tau, d)) = qs;
    *reinterpret_cast<u32x2*>(lds + L_ATT + SK + ((kr >> 4) * 3 + (d >> 5)) * 1024 + frag_pos(kr, d)) = ks;
  }
  unsigned short* l16 = reinterpret_cast<unsigned short*>(lds + L_ATT);
#pragma unroll
  for (int s = 0; s < 6; s++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int d = 16 * s + 4 * g4 + i;
      l16[(SV + ((d >> 4) * 2 + (tau >> 5)) * 1024 + frag_pos(d, tau)) >> 1] = (unsigned short)(bf16_bits(v[4 * s + i]) & keep);
    }
  __syncthreads();
  if (16 * c.w < p.Tv) {
    u32x4 qf[3];
#pragma unroll
    for (int ks = 0; ks < 3; ks++) qf[ks] = lds128(L_ATT + SQ + (c.w * 3 + ks) * 1024 + c.lane * 16);
    unsigned vmask[2][4];
#pragma unroll
    for (int sp = 0; sp < 2; sp++)
#pragma unroll
      for (int e = 0; e < 4; e++) vmask[sp][e] = 0xffffffffu;  // keys past Tv hold zeros
    float mx, ps;
    f32x4 o[6];
    attend<4>(qf, L_ATT + SK, L_ATT + SV, p.Tv, vmask, mx, ps, o);
    const int t = 16 * c.w + c.lr;
    if (t < p.Tv) {
#pragma unroll
      for (int dt = 0; dt < 6; dt++)
        *reinterpret_cast<u32x2*>(p.ws + c.xb + X_ATT + afo(3, t, 16 * dt + 4 * c.lq)) =
            u32x2{pack_bf16x2(o[dt][0], o[dt][1]), pack_bf16x2(o[dt][2], o[dt][3])};
    }
  }
}

// ---- cross attention: context keys 32r..32r+31 of head g (ranks 0..15) --------------------------
// kf: K fragments (key tile kt, k-step ks; tile row 4a + i = key 32 r + 8 a + 4 kt + i); vf: V^T
// fragments (dim tile dt; keys 32 r + 8 lq ..). Both were loaded ahead of the barrier.
__device__ __forceinline__ void stage_catt(const Params& p, const Ctx& c, const u32x4 (&kf)[2][3], const u32x4 (&vf)[6]) {
  if (KPR * c.r >= p.Lk) return;
  const int tau = 16 * c.w + c.lr, g4 = c.lq;
  const bool tv = tau < p.Tv;
  float q[24];
  {
    const int tt = 16 * c.w < p.Tv ? c.w : 0;
    u32x4 r[6];
#pragma unroll
    for (int qq = 0; qq < 6; qq++) r[qq] = ldb128<kCpSc1>(c.ws, c.xb + X_QC + (uint32_t)(((tt * 6 + qq) * 64 + c.lane) * 16));
#pragma unroll
    for (int qq = 0; qq < 6; qq++)
#pragma unroll
      for (int i = 0; i < 4; i++) q[4 * qq + i] = as_f32(r[qq][i]);
  }
  rms96(q);
  const unsigned keep = keep_mask(tv);
#pragma unroll
  for (int s = 0; s < 6; s++) {  // element 4 s + i = dim 16 s + 4 g4 + i: half a fragment slot each
    const int d = 16 * s + 4 * g4;
    const u32x2 qs = pack4(q, s, keep);
    *reinterpret_cast<u32x2*>(lds + L_ATT + ((tau >> 4) * 3 + (d >> 5)) * 1024 + frag_pos(tau, d)) = qs;
  }
  __syncthreads();
  if (16 * c.w >= p.Tv) return;
  u32x4 qf[3];
#pragma unroll
  for (int ks = 0; ks < 3; ks++) qf[ks] = lds128(L_ATT + (c.w * 3 + ks) * 1024 + c.lane * 16);
  const int key0 = KPR * c.r;
  const float qscale = 1.4426950408889634f * 0.10206207261596575f;  // log2(e) / sqrt(96)
  f32x4 s[2];
#pragma unroll
  for (int kt = 0; kt < 2; kt++) {
    f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 3; ks++) a = mfma16(kf[kt][ks], qf[ks], a);
    s[kt] = a;
  }
  float m_ = -1e30f;
#pragma unroll
  for (int kt = 0; kt < 2; kt++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int key = key0 + 8 * c.lq + 4 * kt + i;
      s[kt][i] = key < p.Lk ? s[kt][i] * qscale : -1e30f;
      m_ = fmaxf(m_, s[kt][i]);
    }
  m_ = cols_max(m_);
  float pv[8], ps = 0.f;
#pragma unroll
  for (int kt = 0; kt < 2; kt++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      pv[4 * kt + i] = exp2_w(s[kt][i] - m_);
      ps += pv[4 * kt + i];
    }
  ps = cols_sum(ps);
  const u32x4 pb = {pack_bf16x2(pv[0], pv[1]), pack_bf16x2(pv[2], pv[3]), pack_bf16x2(pv[4], pv[5]),
                    pack_bf16x2(pv[6], pv[7])};
  const int nv = min(max(p.Lk - (key0 + 8 * c.lq), 0), 8);
  unsigned vm[4];
#pragma unroll
  for (int e = 0; e < 4; e++) vm[e] = nv >= 2 * e + 2 ? 0xffffffffu : (nv == 2 * e + 1 ? 0xffffu : 0u);
  const float inv = 1.0f / ps;
  const int t = 16 * c.w + c.lr;
#pragma unroll
  for (int dt = 0; dt < 6; dt++) {
    u32x4 va = vf[dt];
#pragma unroll
    for (int e = 0; e < 4; e++) va[e] &= vm[e];
    const f32x4 o = mfma16(va, pb, f32x4{0.f, 0.f, 0.f, 0.f}) * inv;
    if (t < p.Tv)
      *reinterpret_cast<u32x2*>(p.ws + c.xb + X_CP + ((c.r * TP + t) * HD + 16 * dt + 4 * c.lq) * 2) =
          u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
  }
  if (t < p.Tv && c.lq == 0)
    *reinterpret_cast<f32x2*>(p.ws + c.xb + X_CML + (c.r * TP + t) * 8) = f32x2{m_, ps};
}

// attn_g[token r][d] = sum_c w_c O_c[d], w_c ~ l_c 2^(m_c - M); wave 0, lanes < 48 take dims 2l, 2l+1.
__device__ __forceinline__ void stage_comb(const Params& p, const Ctx& c) {
  const int t = c.r;
  if (t >= p.Tv || c.w != 0) return;
  const int nch = (p.Lk + KPR - 1) / KPR;
  const int d0 = 2 * (c.lane < 48 ? c.lane : 0);
  u32x2 ml[16];
  unsigned v[16];
#pragma unroll
  for (int ch = 0; ch < 16; ch++) {
    const int cc = ch < nch ? ch : 0;
    ml[ch] = ldb64<kCpSc1>(c.ws, c.xb + X_CML + (uint32_t)((cc * TP + t) * 8));
    v[ch] = __builtin_amdgcn_raw_buffer_load_b32(c.ws, c.xb + X_CP + (uint32_t)(((cc * TP + t) * HD + d0) * 2), 0, kCpSc1);
  }
  float M = -1e30f;
#pragma unroll
  for (int ch = 0; ch < 16; ch++)
    if (ch < nch) M = fmaxf(M, as_f32(ml[ch][0]));
  float den = 0.f, a0 = 0.f, a1 = 0.f;
#pragma unroll
  for (int ch = 0; ch < 16; ch++) {
    if (ch >= nch) break;
    const float wc = as_f32(ml[ch][1]) * exp2_w(as_f32(ml[ch][0]) - M);
    den += wc;
    a0 = fmaf(wc, bf_lo(v[ch]), a0);
    a1 = fmaf(wc, bf_hi(v[ch]), a1);
  }
  if (c.lane < 48) {
    const float inv = 1.0f / den;
    *reinterpret_cast<unsigned*>(p.ws + c.xb + X_ATT + afo(3, t, d0)) = pack_bf16x2(a0 * inv, a1 * inv);
  }
}

// gate/up rows 24r.. of the head's slice: K = 768 split over the waves (wf[rt][j] = k-step 6w + j)
// -> LDS -> wave (rt, tt) adds, applies biases and silu(g) u, stores h_g fragments.
__device__ __forceinline__ void stage_gu(const Params& p, const Ctx& c, const u32x4 (&wf)[2][6], const float* bias) {
  f32x4 acc[2][2] = {};
  u32x4 b[2][6];
#pragma unroll
  for (int j = 0; j < 6; j++)
#pragma unroll
    for (int tt = 0; tt < 2; tt++)
      b[tt][j] = ldb128<kCpSc1>(c.ws, c.xb + X_XN + (uint32_t)(((tt * (D / 32) + 6 * c.w + j) * 64 + c.lane) * 16));
#pragma unroll
  for (int j = 0; j < 6; j++)
#pragma unroll
    for (int rt = 0; rt < 2; rt++)
#pragma unroll
      for (int tt = 0; tt < 2; tt++) acc[rt][tt] = mfma16(wf[rt][j], b[tt][j], acc[rt][tt]);
  f32x4* red = reinterpret_cast<f32x4*>(lds + L_RED);
#pragma unroll
  for (int rt = 0; rt < 2; rt++)
#pragma unroll
    for (int tt = 0; tt < 2; tt++) red[((c.w * 2 + rt) * 2 + tt) * 64 + c.lane] = acc[rt][tt];
  __syncthreads();
  const int rt = c.w >> 1, tt = c.w & 1;
  f32x4 sm = (red[((0 * 2 + rt) * 2 + tt) * 64 + c.lane] + red[((1 * 2 + rt) * 2 + tt) * 64 + c.lane]) +
             (red[((2 * 2 + rt) * 2 + tt) * 64 + c.lane] + red[((3 * 2 + rt) * 2 + tt) * 64 + c.lane]);
  if (rt == 1 && c.lq >= 2) return;
  const int rl = 24 * c.r + 16 * rt + 4 * c.lq;  // slice row of v[0]; rows 2f / 2f+1 = gate / up
  sm += *reinterpret_cast<const f32x4*>(bias + rl);
  const int t = 16 * tt + c.lr;
  *reinterpret_cast<unsigned*>(p.ws + c.xb + X_H + afo(384 / 32, t, rl >> 1)) =
      pack_bf16x2(silu(sm[0]) * sm[1], silu(sm[2]) * sm[3]);
}

// ---- the kernel --------------------------------------------------------------------------------
__device__ __forceinline__ void mark(const Params& p, int idx, uint64_t& t0) {
  if (p.stage_cycles && blockIdx.x == 0 && threadIdx.x == 0) {
    const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
    p.stage_cycles[idx] += t1 - t0;
    t0 = t1;
  }
}

__global__ void __launch_bounds__(NTHR, 1) ma2x_kernel(Params p) {
  Ctx c;
  c.g = blockIdx.x & 7;
  c.r = blockIdx.x >> 3;
  c.w = wave_id();
  c.lane = lane_id();
  c.lr = c.lane & 15;
  c.lq = c.lane >> 4;
  c.ws = rsrc_all(p.ws);
  c.xb = OFF_XCD + (uint32_t)c.g * XB;
  c.xflag = reinterpret_cast<uint64_t*>(p.ws + OFF_XFLAG) + c.g * NR * 4;
  c.err = reinterpret_cast<unsigned*>(p.ws + OFF_CTRL + 8);
  const uint64_t seq = ld_flag(reinterpret_cast<const uint64_t*>(p.ws + OFF_CTRL));
  c.e = seq << 32;
  const unsigned* pb = reinterpret_cast<const unsigned*>(p.ws + OFF_CTRL + 12);
  unsigned base0 = __hip_atomic_load(pb, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  unsigned base1 = __hip_atomic_load(pb + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned owner =
      __hip_atomic_load(reinterpret_cast<const unsigned*>(p.ws + kWsOwner), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (threadIdx.x == 0 && xcc_id() != (unsigned)c.g) atomicOr(c.err, kErrXcd);
  if (owner != kOwnerMa2Bs1) {
    // Another kernel used the workspace since this one last did: its data may sit in the exchange
    // buffers with any parity. Clear them (parity 0), restart the parity sequence and pass one
    // grid barrier before the first exchange.
    base0 = base1 = 0;
    for (uint32_t i = blockIdx.x * NTHR + threadIdx.x; i < XP_BYTES / 16; i += NWG * NTHR)
      stb128<kCpSc1>(c.ws, OFF_XP + 16 * i, u32x4{0u, 0u, 0u, 0u});
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    c.e += 1;
    if (c.lane == 0) __hip_atomic_store(c.xflag + c.r * 4 + c.w, c.e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    poll_flags(c.ws, OFF_XFLAG, NX * NR * 4 * 8, c.e, c.err);
    __syncthreads();
  }
  float* xt = reinterpret_cast<float*>(lds + L_XT);
  if (c.w == 0 && c.lane < AD && c.r < p.Tv) xt[c.lane] = p.x_t[c.r * AD + c.lane];
  if (c.r == 0) {  // the RoPE table of the self-attention rank, read every layer
    float* rope = reinterpret_cast<float*>(lds + L_ROPE);
    for (int i = threadIdx.x; i < p.Tv * 48; i += NTHR) {
      rope[i] = p.rope_cos[i];
      rope[TP * 48 + i] = p.rope_sin[i];
    }
  }
  __syncthreads();
  // exchange e uses buffer e & 1; the n-th use of a buffer carries parity (1 + base + n) & 1
  auto buf = [](int e) { return e & 1; };
  auto par = [&](int e) { return (1u + ((e & 1) ? base1 : base0) + (unsigned)(e >> 1)) & 1u; };
  const int NL = p.NL;
  const float dt = 1.0f / (float)p.S;
  uint64_t t0 = __builtin_amdgcn_s_memrealtime();
#pragma unroll 1
  for (int step = 0; step < p.S; step++) {
#pragma unroll 1
    for (int l = 0; l < NL; l++) {
      asm volatile("" : "+v"(c.lane), "+v"(c.lr), "+v"(c.lq));
      const int li = step * NL + l;
      const float* mo = p.mods + ((size_t)step * NL + l) * 9 * D;
      const int e0 = 3 * li, e1 = e0 + 1, e2 = e0 + 2;
      // N_msa, with the QKV weights of ranks 0..17 in flight
      u32x4 wq[6];
      if (c.r < 18) {
        const int row = (c.r / 6) * D + HD * c.g + 16 * (c.r % 6) + c.lr;
        const bf16* W = p.w_qkv + (size_t)l * QKVN * D;
#pragma unroll
        for (int j = 0; j < 6; j++) wq[j] = wfrag(W, D, row, 32 * (6 * c.w + j), c.lq);
      }
      if (l == 0)
        stage_norm<0>(p, c, 0, 0u, nullptr, nullptr, mo, mo + D, 0.f);
      else
        stage_norm<1>(p, c, buf(e0 - 1), par(e0 - 1), p.b_dn + (size_t)(l - 1) * D, mo - 9 * D + 8 * D, mo, mo + D,
                      0.f);
      mark(p, 0, t0);
      xarrive(c);
      xwait(c);
      mark(p, 15, t0);
      // QKV
      if (c.r < 18)
        gemm16(p, c, wq, X_QKV, 3, 96 * (c.r / 6) + 16 * (c.r % 6),
               p.b_qkv + (size_t)l * QKVN + (c.r / 6) * D + HD * c.g + 16 * (c.r % 6));
      mark(p, 1, t0);
      xarrive(c);
      u32x4 wso[3];
      {
        const bf16* W = p.w_so + (size_t)l * D * D;
        const int row = row24(24 * c.r, c.w >> 1, c.lr);
#pragma unroll
        for (int j = 0; j < 3; j++) wso[j] = wfrag(W, D, row, HD * c.g + 32 * j, c.lq);
      }
      xwait(c);
      mark(p, 15, t0);
      // SATT
      if (c.r == 0) stage_satt(p, c);
      mark(p, 2, t0);
      xarrive(c);
      xwait(c);
      mark(p, 15, t0);
      // SO -> exchange e0
      proj24<3>(p, c, wso, X_ATT, 3, buf(e0), par(e0));
      mark(p, 3, t0);
      // N_mca, with the CQ weights (ranks 0..5) and this rank's context keys/values in flight
      u32x4 wc[6], kf[2][3], vf[6];
      if (c.r < 6) {
        const bf16* W = p.w_cq + (size_t)l * D * D;
        const int row = HD * c.g + 16 * c.r + c.lr;
#pragma unroll
        for (int j = 0; j < 6; j++) wc[j] = wfrag(W, D, row, 32 * (6 * c.w + j), c.lq);
      }
      if (KPR * c.r < p.Lk && c.w < 2) {
        const bf16* K = p.kctx + (size_t)l * p.Lkmax * D;
        const bf16* V = p.vtctx + (size_t)l * D * p.Lkmax;
#pragma unroll
        for (int kt = 0; kt < 2; kt++) {
          int key = KPR * c.r + 8 * (c.lr >> 2) + 4 * kt + (c.lr & 3);
          if (key >= p.Lk) key = 0;
#pragma unroll
          for (int ks = 0; ks < 3; ks++) kf[kt][ks] = wfrag(K, D, key, HD * c.g + 32 * ks, c.lq);
        }
        int kg = KPR * c.r + 8 * c.lq;
        if (kg >= p.Lk) kg = 0;
#pragma unroll
        for (int dt2 = 0; dt2 < 6; dt2++)
          vf[dt2] = *reinterpret_cast<const u32x4*>(V + (size_t)(HD * c.g + 16 * dt2 + c.lr) * p.Lkmax + kg);
      }
      stage_norm<1>(p, c, buf(e0), par(e0), p.b_so + (size_t)l * D, mo + 2 * D, mo + 3 * D, mo + 4 * D, 0.f);
      mark(p, 4, t0);
      xarrive(c);
      xwait(c);
      mark(p, 15, t0);
      // CQ
      if (c.r < 6) gemm16(p, c, wc, X_QC, 1, 16 * c.r, p.b_cq + (size_t)l * D + HD * c.g + 16 * c.r);
      mark(p, 5, t0);
      xarrive(c);
      xwait(c);
      mark(p, 15, t0);
      // CATT
      stage_catt(p, c, kf, vf);
      mark(p, 6, t0);
      xarrive(c);
      xwait(c);
      mark(p, 15, t0);
      // COMB, with the CO weights in flight
      stage_comb(p, c);
      mark(p, 7, t0);
      xarrive(c);
      u32x4 wco[3];
      {
        const bf16* W = p.w_co + (size_t)l * D * D;
        const int row = row24(24 * c.r, c.w >> 1, c.lr);
#pragma unroll
        for (int j = 0; j < 3; j++) wco[j] = wfrag(W, D, row, HD * c.g + 32 * j, c.lq);
      }
      xwait(c);
      mark(p, 15, t0);
      // CO -> exchange e1
      proj24<3>(p, c, wco, X_ATT, 3, buf(e1), par(e1));
      mark(p, 8, t0);
      // N_mlp, with the gate/up weights in flight
      u32x4 wg[2][6];
      {
        const bf16* W = p.w_gu + (size_t)l * GUN * D;
#pragma unroll
        for (int rt = 0; rt < 2; rt++) {
          const int row = 2 * 384 * c.g + row24(24 * c.r, rt, c.lr);
#pragma unroll
          for (int j = 0; j < 6; j++) wg[rt][j] = wfrag(W, D, row, 32 * (6 * c.w + j), c.lq);
        }
      }
      stage_norm<1>(p, c, buf(e1), par(e1), p.b_co + (size_t)l * D, mo + 5 * D, mo + 6 * D, mo + 7 * D, 0.f);
      mark(p, 9, t0);
      xarrive(c);
      xwait(c);
      mark(p, 15, t0);
      // GU, then the down weights in flight
      stage_gu(p, c, wg, p.b_gu + (size_t)l * GUN + 2 * 384 * c.g);
      mark(p, 10, t0);
      xarrive(c);
      u32x4 wd[12];
      {
        const bf16* W = p.w_dn + (size_t)l * D * FF;
        const int row = row24(24 * c.r, c.w >> 1, c.lr);
#pragma unroll
        for (int j = 0; j < 12; j++) wd[j] = wfrag(W, FF, row, 384 * c.g + 32 * j, c.lq);
      }
      xwait(c);
      mark(p, 15, t0);
      // DN -> exchange e2
      proj24<12>(p, c, wd, X_H, 12, buf(e2), par(e2));
      mark(p, 11, t0);
    }
    const int el = 3 * (step * NL + NL - 1) + 2;
    const float* ml = p.mods + ((size_t)step * NL + NL - 1) * 9 * D;
    const float* mf = p.mod_final + (size_t)step * 2 * D;
    stage_norm<2>(p, c, buf(el), par(el), p.b_dn + (size_t)(NL - 1) * D, ml + 8 * D, mf, mf + D, dt);
    mark(p, 12, t0);
  }
  if (c.g == 0 && c.w == 0 && c.lane < AD && c.r < p.Tv) p.x_t[c.r * AD + c.lane] = xt[c.lane];
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    const unsigned n = 3u * (unsigned)(p.S * NL);  // exchanges in this launch
    unsigned* pw = reinterpret_cast<unsigned*>(p.ws + OFF_CTRL + 12);
    __hip_atomic_store(pw, (base0 + (n + 1) / 2) & 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(pw + 1, (base1 + n / 2) & 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(reinterpret_cast<unsigned*>(p.ws + kWsOwner), kOwnerMa2Bs1, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p.ws + OFF_CTRL), seq + 1, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace ma2x

// ---- host: batch-1 launch of fa_ma2_flow (argument checks done by the caller in ma2.hip) -------
bool ma2_bs1_eligible(int batch, int Tv, int Lkmax) {
  return batch == 1 && Tv <= ma2x::TP && Lkmax <= ma2x::MAX_LK;
}
size_t ma2_bs1_workspace_bytes() { return ma2x::WS_BYTES; }

int ma2_bs1_launch(const fa_ma2_args* a, fa_stream_t stream) {
  using namespace fa::ma2x;
  if (a->workspace_bytes < WS_BYTES)
    return host::fail(FA_ERR_INVALID_ARG, "fa_ma2_flow: workspace_bytes=%zu < required %u", a->workspace_bytes,
                      (unsigned)WS_BYTES);
  int rc = host::check_device((const void*)ma2x_kernel, NTHR, LDS_BYTES, NWG, "fa_ma2_flow");
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
  p.NL = a->num_layers;
  p.Lk = a->Lk;
  p.Lkmax = a->Lkmax;
  p.Tv = a->Tv;
  p.adim = a->adim;
  p.S = a->num_steps;
  void* args[] = {&p};
  return host::coop_launch((const void*)ma2x_kernel, NWG, NTHR, args, LDS_BYTES, stream, "fa_ma2_flow");
}

}  // namespace fa
