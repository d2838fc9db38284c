// pi0.5 action-expert denoise loop, batch 1: the whole S-step Euler loop in ONE cooperative
// launch of 256 workgroups (one per CU) x 256 threads (4 waves, one per SIMD) on gfx950.
//
// Work decomposition (XCD-aware; XCD g = blockIdx % 8, rank r = blockIdx / 8 in 0..31):
//   XCD g owns query head g (attention), the MLP columns f in [512g, 512g+512) and the
//   K-windows g of the O and down projections. Everything a head/F-slice needs stays inside
//   the XCD's L2; only the O and down partial sums cross XCDs. Per layer:
//     N1  [XCD]  QKV  [XCD]  ATT  [XCD]  COMB  [XCD]  O  [GRID]  N2  [XCD]  GU  [XCD]  DN  [GRID]
//   (the reference runs 9 grid-wide barriers per layer: src/pi05/mk6.cu:301-497).
//   N1/N2/FINAL: rank r owns tokens r and r+32 of its XCD: combine the 8 XCD partials, gated
//        residual, adaRMS -> bf16 operand. The residual x and x_t live in that CU's LDS.
//   QKV: 768 rows per XCD (q rows of head g + all k and v rows), 24 rows per CU, RoPE epilogue.
//   ATT: head g, keys split into 32 chunks (one per rank); MFMA S^T = K Q^T, online softmax,
//        O^T = V^T P^T; partial (O, m, l) per chunk.
//   COMB: flash-decoding combine of the 32 chunk partials -> attn_g (bf16).
//   O:   W_o[32r..32r+32, 256g..256g+256) x attn_g -> partial o_g (sc1, cross-XCD).
//   GU:  32 interleaved gate/up rows per CU -> gelu_tanh(g)*u -> h_g (bf16, XCD-private).
//   DN:  W_d[32r..32r+32, 512g..512g+512) x h_g -> partial z_g (sc1, cross-XCD).
// GEMMs: v_mfma_f32_16x16x32_bf16 with weight rows as the A operand (16 rows x 32 k per
// fragment, one 16-byte load per lane) and tokens as B; the 4 waves split K and reduce in LDS.
// Weight fragments of the next GEMM stage are issued after a workgroup publishes its barrier
// epoch and before it waits, so HBM streaming overlaps the barrier.
#include "fa_device.h"
#include "../../include/flashact_mi355x.h"
#include "fa_host.h"

namespace fa {
namespace pi05 {

constexpr int D = 1024, HD = 256, AD = 32;
constexpr int NX = 8, NR = 32, NWG = 256, NTH = 256, TP = 64;
constexpr int NCH = 32;  // attention key chunks per head (= ranks)
constexpr uint32_t LDS_BYTES = 96 * 1024;  // > 80 KB forces one workgroup per CU
constexpr uint32_t OOB = 0x80000000u;      // buffer offset past every resource: loads return 0

// workspace layout (bytes)
constexpr uint32_t OFF_CTRL = 0;          // u64 seq, u32 err
constexpr uint32_t OFF_XFLAG = 256;       // [8][32] u64
constexpr uint32_t OFF_GFLAG = 2304;      // [8] u64
constexpr uint32_t OFF_XN = 4096;                                   // [8][64][1024] bf16
constexpr uint32_t OFF_Q = OFF_XN + NX * TP * D * 2;                // [8][64][256] bf16
constexpr uint32_t OFF_ATTP = OFF_Q + NX * TP * HD * 2;             // [8][32][64][256] f32
constexpr uint32_t OFF_ATTML = OFF_ATTP + NX * NCH * TP * HD * 4;   // [8][32][64][2] f32
constexpr uint32_t OFF_ATTN = OFF_ATTML + NX * NCH * TP * 2 * 4;    // [8][64][256] bf16
constexpr uint32_t OFF_H = OFF_ATTN + NX * TP * HD * 2;             // [8][64][512] bf16
constexpr uint32_t OFF_OPART = OFF_H + NX * TP * 512 * 2;           // [8][64][1024] f32
constexpr uint32_t OFF_ZPART = OFF_OPART + NX * TP * D * 4;         // [8][64][1024] f32
constexpr uint32_t WS_BYTES = OFF_ZPART + NX * TP * D * 4;

struct Params {
  const bf16* w1;
  const bf16* wo;
  const bf16* w2;
  const bf16* w3;
  const float* mods;
  const float* mod_final;
  const float* rope_cos;
  const float* rope_sin;
  const float* w_ain;
  const float* b_ain;
  const float* w_aout;
  const float* b_aout;
  bf16* kcache;
  bf16* vtcache;
  float* x_t;
  unsigned long long* stage_cycles;
  unsigned char* ws;
  int NL, Lp, Lmax, S, Tv, xt_rows;
};

// LDS map (floats)
constexpr int L_XRES = 0;                 // [2][1024] residual stream of my two tokens
constexpr int L_XT = L_XRES + 2 * D;      // [2][32]   x_t of my two tokens
constexpr int L_WSUM = L_XT + 2 * AD;     // [16]      cross-wave partial sums
constexpr int L_CW = L_WSUM + 16;         // [2][32]   combine weights
constexpr int L_HFIN = L_CW + 64;         // [2][1024] final-norm output
constexpr int L_RED = L_HFIN + 2 * D;     // [4 waves][8 frags][64 lanes] f32x4 (32 KB)

struct Ctx {
  int g, r, tid, lane, wave, lr, lq;
  rsrc_t ws;      // whole workspace
  rsrc_t kc, vc;  // caches
  float* lds;
  f32x4* red;
};

__device__ __forceinline__ void mark(const Params& p, const Ctx& c, int idx, uint64_t& t0) {
  if (p.stage_cycles && blockIdx.x == 0 && threadIdx.x == 0) {
    uint64_t now = __builtin_amdgcn_s_memrealtime();
    p.stage_cycles[idx] += now - t0;  // slots 0-8: stage work, 9: XCD waits, 10: grid waits
    t0 = now;
  }
}

// ---------------------------------------------------------------- GEMM core
// acc[rt][tt] = sum over this wave's K range of W[rows rt*16+lr][k] * X[token tt*16+lr][k].
// wf: weight fragments already in registers. X fragments are read here with sc1 loads from
// the XCD-private operand at byte offset xoff (row t=lr, k = wave start + 8*lq), rows xrow bytes.
template <int RT, int KS>
__device__ __forceinline__ void gemm_core(f32x4 (&acc)[RT][4], const u32x4 (&wf)[RT][KS], const Ctx& c, uint32_t xoff,
                                          uint32_t xrow, int Tv) {
  u32x4 xf[4][KS];
#pragma unroll
  for (int tt = 0; tt < 4; tt++) {
    const uint32_t base = tt * 16 + c.lr < Tv ? xoff + tt * 16 * xrow : OOB;
#pragma unroll
    for (int ks = 0; ks < KS; ks++) xf[tt][ks] = ldb128<kCpSc1>(c.ws, base + ks * 64);
  }
#pragma unroll
  for (int rt = 0; rt < RT; rt++)
#pragma unroll
    for (int tt = 0; tt < 4; tt++) acc[rt][tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < KS; ks++)
#pragma unroll
    for (int rt = 0; rt < RT; rt++)
#pragma unroll
      for (int tt = 0; tt < 4; tt++) acc[rt][tt] = mfma16(wf[rt][ks], xf[tt][ks], acc[rt][tt]);
}

// Cross-wave K reduction: after this, reduce_get(rt) returns the full sum of fragment
// (rt, token tile = this wave).
template <int RT>
__device__ __forceinline__ void reduce_put(const Ctx& c, const f32x4 (&acc)[RT][4]) {
#pragma unroll
  for (int rt = 0; rt < RT; rt++)
#pragma unroll
    for (int tt = 0; tt < 4; tt++) c.red[((c.wave * RT + rt) * 4 + tt) * 64 + c.lane] = acc[rt][tt];
  __syncthreads();
}
template <int RT>
__device__ __forceinline__ f32x4 reduce_get(const Ctx& c, int rt) {
  f32x4 s = c.red[((0 * RT + rt) * 4 + c.wave) * 64 + c.lane];
#pragma unroll
  for (int w = 1; w < 4; w++) s += c.red[((w * RT + rt) * 4 + c.wave) * 64 + c.lane];
  return s;
}

// ---------------------------------------------------------------- norm stages
// MODE 0: x = embed(x_t) (layer 0).  MODE 1: x += gate * sum_g part_g.  MODE 2: as 1, final norm.
// Writes xres (LDS) and xn_g (bf16) or, for MODE 2, the fp32 normalised rows to LDS.
template <int MODE>
__device__ __forceinline__ void stage_norm(const Params& p, const Ctx& c, uint32_t part_off, const float* gate,
                                           const float* scale, const float* shift) {
  float* xres = c.lds + L_XRES;
  float* xt = c.lds + L_XT;
  float* wsum = c.lds + L_WSUM;
  const int d0 = c.tid * 4;
  f32x4 xv[2];
  float ss[2];
  u32x4 part[2][NX];
  if (MODE != 0) {
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int t = c.r + 32 * j;
#pragma unroll
      for (int gg = 0; gg < NX; gg++)
        part[j][gg] = ldb128<kCpSc1>(c.ws, t < p.Tv ? part_off + ((gg * TP + t) * D + d0) * 4 : OOB);
    }
  }
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int t = c.r + 32 * j;
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (t < p.Tv) {
      if (MODE == 0) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float* w = p.w_ain + (d0 + i) * AD;
          float a = p.b_ain[d0 + i];
#pragma unroll 8
          for (int k = 0; k < AD; k++) a = fmaf(w[k], xt[j * AD + k], a);
          v[i] = a;
        }
      } else {
        f32x4 sum = as_f32x4(part[j][0]);
#pragma unroll
        for (int gg = 1; gg < NX; gg++) sum += as_f32x4(part[j][gg]);
        const f32x4 gt = *reinterpret_cast<const f32x4*>(gate + d0);
        const f32x4 xo = *reinterpret_cast<const f32x4*>(xres + j * D + d0);
        v = xo + gt * sum;
      }
    }
    xv[j] = v;
    ss[j] = v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
  }
#pragma unroll
  for (int j = 0; j < 2; j++) {
    float s = wave_sum(ss[j]);
    if (c.lane == 0) wsum[c.wave * 2 + j] = s;
  }
  __syncthreads();
  const f32x4 sc = *reinterpret_cast<const f32x4*>(scale + d0);
  const f32x4 sh = *reinterpret_cast<const f32x4*>(shift + d0);
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int t = c.r + 32 * j;
    if (t >= p.Tv) continue;
    const float tot = (wsum[0 * 2 + j] + wsum[1 * 2 + j]) + (wsum[2 * 2 + j] + wsum[3 * 2 + j]);
    const float rr = rsqrtf(tot / (float)D + 1e-6f);
    *reinterpret_cast<f32x4*>(xres + j * D + d0) = xv[j];
    f32x4 h;
#pragma unroll
    for (int i = 0; i < 4; i++) h[i] = xv[j][i] * rr * (1.0f + sc[i]) + sh[i];
    if (MODE == 2) {
      *reinterpret_cast<f32x4*>(c.lds + L_HFIN + j * D + d0) = h;
    } else {
      u32x2 pk = {pack_bf16x2(h[0], h[1]), pack_bf16x2(h[2], h[3])};
      *reinterpret_cast<u32x2*>(p.ws + OFF_XN + ((c.g * TP + t) * D + d0) * 2) = pk;
    }
  }
  __syncthreads();
}

// action_out + Euler update of my two tokens (after stage_norm<2>)
__device__ __forceinline__ void stage_action(const Params& p, const Ctx& c, float dt) {
  const float* hf = c.lds + L_HFIN;
  float* xt = c.lds + L_XT;
#pragma unroll 1
  for (int ai = 0; ai < 8; ai++) {
    const int a = c.wave * 8 + ai;
    float acc[2] = {0.f, 0.f};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int d = k * 256 + c.lane * 4;
      const f32x4 w = *reinterpret_cast<const f32x4*>(p.w_aout + a * D + d);
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const f32x4 h = *reinterpret_cast<const f32x4*>(hf + j * D + d);
        acc[j] += w[0] * h[0] + w[1] * h[1] + w[2] * h[2] + w[3] * h[3];
      }
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const float v = wave_sum(acc[j]);
      if (c.lane == 0 && c.r + 32 * j < p.Tv) xt[j * AD + a] += dt * (v + p.b_aout[a]);
    }
  }
  __syncthreads();
}

// ---------------------------------------------------------------- QKV
__device__ __forceinline__ int qkv_row(int g, int vr) {
  return vr < 256 ? 256 * g + vr : (vr < 512 ? 2048 + (vr - 256) : 2304 + (vr - 512));
}

__device__ __forceinline__ void load_w_qkv(const Params& p, const Ctx& c, int l, u32x4 (&w)[2][8]) {
#pragma unroll
  for (int rt = 0; rt < 2; rt++) {
    const bool ok = rt == 0 || c.lr < 8;
    const int row = qkv_row(c.g, 24 * c.r + rt * 16 + c.lr);
    const bf16* base = p.w1 + ((size_t)l * 2560 + (ok ? row : 0)) * D + c.wave * 256 + c.lq * 8;
#pragma unroll
    for (int ks = 0; ks < 8; ks++) w[rt][ks] = ok ? ld_stream128(base + ks * 32) : u32x4{0, 0, 0, 0};
  }
}

__device__ __forceinline__ void stage_qkv(const Params& p, const Ctx& c, int l, const u32x4 (&w)[2][8]) {
  f32x4 acc[2][4];
  gemm_core<2, 8>(acc, w, c, OFF_XN + ((c.g * TP + c.lr) * D + c.wave * 256 + c.lq * 8) * 2, D * 2, p.Tv);
  reduce_put<2>(c, acc);
  const int t = c.wave * 16 + c.lr;
#pragma unroll
  for (int rt = 0; rt < 2; rt++) {
    const f32x4 v = reduce_get<2>(c, rt);
    if (rt == 1 && c.lq >= 2) continue;  // rows 24r+24.. belong to the next rank
    if (t >= p.Tv) continue;
    const int vr0 = 24 * c.r + rt * 16 + 4 * c.lq;
    if (vr0 < 512) {
      const int j = (vr0 & 255) >> 1;  // RoPE pair index within the head
      const float* cs = p.rope_cos + t * 128 + j;
      const float* sn = p.rope_sin + t * 128 + j;
      const float lo0 = v[0] * cs[0] - v[1] * sn[0], hi0 = v[1] * cs[0] + v[0] * sn[0];
      const float lo1 = v[2] * cs[1] - v[3] * sn[1], hi1 = v[3] * cs[1] + v[2] * sn[1];
      const unsigned plo = pack_bf16x2(lo0, lo1), phi = pack_bf16x2(hi0, hi1);
      if (vr0 < 256) {
        const uint32_t off = OFF_Q + ((c.g * TP + t) * HD + j) * 2;
        *reinterpret_cast<unsigned*>(p.ws + off) = plo;
        *reinterpret_cast<unsigned*>(p.ws + off + 256) = phi;
      } else {
        // Suffix keys go to the caller's cache (the reference's output contract). Every XCD
        // writes the same values and reads back its own L2 copy in the attention stage.
        bf16* kr = p.kcache + ((size_t)l * p.Lmax + p.Lp + t) * HD;
        *reinterpret_cast<unsigned*>(kr + j) = plo;
        *reinterpret_cast<unsigned*>(kr + j + 128) = phi;
      }
    } else {
      const int d = vr0 - 512;
      bf16* vr = p.vtcache + ((size_t)l * HD + d) * p.Lmax + p.Lp + t;
#pragma unroll
      for (int i = 0; i < 4; i++) vr[(size_t)i * p.Lmax] = (bf16)v[i];
    }
  }
}

// ---------------------------------------------------------------- attention partials
// Head g, keys [r*C, r*C+C): prefix keys and this step's suffix keys both come from the caches.
// Per 32-key block every K row fragment and V^T fragment is issued before the first MFMA.
__device__ __forceinline__ void stage_att(const Params& p, const Ctx& c, int l) {
  const int Ltot = p.Lp + p.Tv;
  const int C = 32 * ((Ltot + 32 * NCH - 1) / (32 * NCH));
  const int kbeg = c.r * C;
  const int kend = min(kbeg + C, Ltot);
  const int t = c.wave * 16 + c.lr;
  const bool tok_ok = t < p.Tv;
  const float qscale = 1.4426950408889634f / 16.0f;  // log2(e) / sqrt(256)

  u32x4 qf[8];
  {
    const uint32_t qb = tok_ok ? OFF_Q + ((c.g * TP + t) * HD + c.lq * 8) * 2 : OOB;
#pragma unroll
    for (int ks = 0; ks < 8; ks++) qf[ks] = ldb128<kCpSc1>(c.ws, qb + ks * 64);
  }
  float m = -1e30f, lsum = 0.f;
  f32x4 o[16];
#pragma unroll
  for (int dt = 0; dt < 16; dt++) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};

  const uint32_t kl = (uint32_t)l * p.Lmax * HD * 2;  // layer base, kcache [Lmax][256]
  const uint32_t vl = (uint32_t)l * HD * p.Lmax * 2;  // layer base, vtcache [256][Lmax]
#pragma unroll 1
  for (int kb = kbeg; kb < kend; kb += 32) {
    u32x4 kf[2][8];
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
      const int key = kb + kt * 16 + c.lr;
      const uint32_t rb = key < kend ? kl + key * HD * 2 + c.lq * 16 : OOB;
#pragma unroll
      for (int ks = 0; ks < 8; ks++) kf[kt][ks] = ldb128<kCpSc1>(c.kc, rb + ks * 64);
    }
    // V^T fragments: dim 16dt+lr, keys kg0 = kb+4lq+(0..3) and kg1 = kb+16+4lq+(0..3).
    // The first half is issued with K; the second after the S MFMAs release the K registers.
    const int kg0 = kb + c.lq * 4, kg1 = kg0 + 16;
    const uint32_t vo0 = kg0 < kend ? vl + c.lr * p.Lmax * 2 + kg0 * 2 : OOB;
    const uint32_t vo1 = kg1 < kend ? vl + c.lr * p.Lmax * 2 + kg1 * 2 : OOB;
    const uint32_t vstep = 16 * p.Lmax * 2;  // 16 dims
    u32x2 vf[16][2];
#pragma unroll
    for (int dt = 0; dt < 8; dt++) {
      vf[dt][0] = ldb64<kCpSc1>(c.vc, vo0 + (vo0 == OOB ? 0 : dt * vstep));
      vf[dt][1] = ldb64<kCpSc1>(c.vc, vo1 + (vo1 == OOB ? 0 : dt * vstep));
    }
    // zero V elements of keys >= kend inside a partially valid 4-key group
    unsigned vm[2][2];
#pragma unroll
    for (int h2 = 0; h2 < 2; h2++) {
      const int nv = min(max(kend - (h2 ? kg1 : kg0), 0), 4);
      vm[h2][0] = nv >= 2 ? 0xffffffffu : (nv == 1 ? 0xffffu : 0u);
      vm[h2][1] = nv >= 4 ? 0xffffffffu : (nv == 3 ? 0xffffu : 0u);
    }
    f32x4 s[2];
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
      f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 8; ks++) a = mfma16(kf[kt][ks], qf[ks], a);
      s[kt] = a;
    }
#pragma unroll
    for (int dt = 8; dt < 16; dt++) {
      vf[dt][0] = ldb64<kCpSc1>(c.vc, vo0 + (vo0 == OOB ? 0 : dt * vstep));
      vf[dt][1] = ldb64<kCpSc1>(c.vc, vo1 + (vo1 == OOB ? 0 : dt * vstep));
    }
    // lane holds S^T[key kb + 16kt + 4lq + i][token lr]
    float bmax = -1e30f;
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int key = kb + kt * 16 + c.lq * 4 + i;
        s[kt][i] = key < kend ? s[kt][i] * qscale : -1e30f;
        bmax = fmaxf(bmax, s[kt][i]);
      }
    bmax = fmaxf(bmax, __shfl_xor(bmax, 16, 64));
    bmax = fmaxf(bmax, __shfl_xor(bmax, 32, 64));
    const float mnew = fmaxf(m, bmax);
    const float alpha = exp2f(m - mnew);
    m = mnew;
    float psum = 0.f;
    unsigned pk[4];
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
      float pv[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        pv[i] = exp2f(s[kt][i] - m);
        psum += pv[i];
      }
      pk[kt * 2 + 0] = pack_bf16x2(pv[0], pv[1]);
      pk[kt * 2 + 1] = pack_bf16x2(pv[2], pv[3]);
    }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    lsum = lsum * alpha + psum;
    // B operand P^T: k-slot 8lq+i <-> key kg0+i (i<4), kg1+(i-4) (i>=4)
    const u32x4 pb = {pk[0], pk[1], pk[2], pk[3]};
#pragma unroll
    for (int dt = 0; dt < 16; dt++) {
      const u32x4 va = {vf[dt][0][0] & vm[0][0], vf[dt][0][1] & vm[0][1], vf[dt][1][0] & vm[1][0],
                        vf[dt][1][1] & vm[1][1]};
      o[dt] = mfma16(va, pb, o[dt] * alpha);
    }
  }
  // lane holds O^T[dim 16dt + 4lq + i][token lr]
  if (tok_ok) {
    const uint32_t base = OFF_ATTP + (((c.g * NCH + c.r) * TP + t) * HD + c.lq * 4) * 4;
#pragma unroll
    for (int dt = 0; dt < 16; dt++) *reinterpret_cast<f32x4*>(p.ws + base + dt * 64) = o[dt];
    if (c.lq == 0) {
      f32x2 ml = {m, lsum};
      *reinterpret_cast<f32x2*>(p.ws + OFF_ATTML + (((c.g * NCH + c.r) * TP + t) * 2) * 4) = ml;
    }
  }
}

// ---------------------------------------------------------------- combine
// attn_g[t] = sum_ch 2^(m_ch - M) O_ch[t] / sum_ch 2^(m_ch - M) l_ch for my tokens r, r+32.
__device__ __forceinline__ void stage_comb(const Params& p, const Ctx& c) {
  float* cw = c.lds + L_CW;
  float* red2 = reinterpret_cast<float*>(c.red);  // [4 chunk groups][2 tokens][256]
  if (c.tid < 64) {
    const int j = c.tid >> 5, ch = c.tid & 31;
    const int t = c.r + 32 * j;
    const u32x2 v = ldb64<kCpSc1>(c.ws, t < p.Tv ? OFF_ATTML + (((c.g * NCH + ch) * TP + t) * 2) * 4 : OOB);
    const float mc = t < p.Tv ? as_f32(v[0]) : -1e30f;
    const float lc = as_f32(v[1]);
    float M = mc;
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
    const float wgt = exp2f(mc - M);
    float L = wgt * lc;
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) L += __shfl_xor(L, o, 64);
    cw[j * 32 + ch] = (t < p.Tv) ? wgt / L : 0.f;
  }
  const int q = c.tid & 63, cg = c.tid >> 6;  // dims 4q..4q+3, chunks 8cg..8cg+7
  u32x4 buf[2][8];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    const int t = c.r + 32 * j;
#pragma unroll
    for (int k = 0; k < 8; k++)
      buf[j][k] = ldb128<kCpSc1>(
          c.ws, t < p.Tv ? OFF_ATTP + (((c.g * NCH + cg * 8 + k) * TP + t) * HD + 4 * q) * 4 : OOB);
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 2; j++) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < 8; k++) acc += cw[j * 32 + cg * 8 + k] * as_f32x4(buf[j][k]);
    *reinterpret_cast<f32x4*>(red2 + (cg * 2 + j) * HD + 4 * q) = acc;
  }
  __syncthreads();
  if (c.tid < 128) {
    const int j = c.tid >> 6, t = c.r + 32 * j;
    if (t < p.Tv) {
      f32x4 a = *reinterpret_cast<const f32x4*>(red2 + (0 * 2 + j) * HD + 4 * q);
#pragma unroll
      for (int g2 = 1; g2 < 4; g2++) a += *reinterpret_cast<const f32x4*>(red2 + (g2 * 2 + j) * HD + 4 * q);
      const u32x2 pk = {pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3])};
      *reinterpret_cast<u32x2*>(p.ws + OFF_ATTN + ((c.g * TP + t) * HD + 4 * q) * 2) = pk;
    }
  }
}

// ---------------------------------------------------------------- O projection (K-window g)
__device__ __forceinline__ void load_w_o(const Params& p, const Ctx& c, int l, u32x4 (&w)[2][2]) {
#pragma unroll
  for (int rt = 0; rt < 2; rt++) {
    const bf16* base = p.wo + ((size_t)l * D + 32 * c.r + rt * 16 + c.lr) * 2048 + 256 * c.g + c.wave * 64 + c.lq * 8;
#pragma unroll
    for (int ks = 0; ks < 2; ks++) w[rt][ks] = ld_stream128(base + ks * 32);
  }
}

__device__ __forceinline__ void stage_oproj(const Params& p, const Ctx& c, const u32x4 (&w)[2][2]) {
  f32x4 acc[2][4];
  gemm_core<2, 2>(acc, w, c, OFF_ATTN + ((c.g * TP + c.lr) * HD + c.wave * 64 + c.lq * 8) * 2, HD * 2, p.Tv);
  reduce_put<2>(c, acc);
  const int t = c.wave * 16 + c.lr;
#pragma unroll
  for (int rt = 0; rt < 2; rt++) {
    const f32x4 v = reduce_get<2>(c, rt);
    if (t < p.Tv)
      stb128<kCpSc1>(c.ws, OFF_OPART + ((c.g * TP + t) * D + 32 * c.r + rt * 16 + 4 * c.lq) * 4,
                     as_u32x4(v));
  }
}

// ---------------------------------------------------------------- gate/up (F-slice g)
__device__ __forceinline__ void load_w_gu(const Params& p, const Ctx& c, int l, u32x4 (&w)[2][8]) {
#pragma unroll
  for (int rt = 0; rt < 2; rt++) {
    const bf16* base = p.w2 + ((size_t)l * 8192 + 1024 * c.g + 32 * c.r + rt * 16 + c.lr) * D + c.wave * 256 + c.lq * 8;
#pragma unroll
    for (int ks = 0; ks < 8; ks++) w[rt][ks] = ld_stream128(base + ks * 32);
  }
}

__device__ __forceinline__ void stage_gu(const Params& p, const Ctx& c, const u32x4 (&w)[2][8]) {
  f32x4 acc[2][4];
  gemm_core<2, 8>(acc, w, c, OFF_XN + ((c.g * TP + c.lr) * D + c.wave * 256 + c.lq * 8) * 2, D * 2, p.Tv);
  reduce_put<2>(c, acc);
  const int t = c.wave * 16 + c.lr;
#pragma unroll
  for (int rt = 0; rt < 2; rt++) {
    const f32x4 v = reduce_get<2>(c, rt);
    if (t >= p.Tv) continue;
    const int f0 = 16 * c.r + 8 * rt + 2 * c.lq;  // local MLP column of rows (gate, up) pairs
    *reinterpret_cast<unsigned*>(p.ws + OFF_H + ((c.g * TP + t) * 512 + f0) * 2) =
        pack_bf16x2(gelu_tanh(v[0]) * v[1], gelu_tanh(v[2]) * v[3]);
  }
}

// ---------------------------------------------------------------- down (K-window g)
__device__ __forceinline__ void load_w_dn(const Params& p, const Ctx& c, int l, u32x4 (&w)[2][4]) {
#pragma unroll
  for (int rt = 0; rt < 2; rt++) {
    const bf16* base = p.w3 + ((size_t)l * D + 32 * c.r + rt * 16 + c.lr) * 4096 + 512 * c.g + c.wave * 128 + c.lq * 8;
#pragma unroll
    for (int ks = 0; ks < 4; ks++) w[rt][ks] = ld_stream128(base + ks * 32);
  }
}

__device__ __forceinline__ void stage_dn(const Params& p, const Ctx& c, const u32x4 (&w)[2][4]) {
  f32x4 acc[2][4];
  gemm_core<2, 4>(acc, w, c, OFF_H + ((c.g * TP + c.lr) * 512 + c.wave * 128 + c.lq * 8) * 2, 512 * 2, p.Tv);
  reduce_put<2>(c, acc);
  const int t = c.wave * 16 + c.lr;
#pragma unroll
  for (int rt = 0; rt < 2; rt++) {
    const f32x4 v = reduce_get<2>(c, rt);
    if (t < p.Tv)
      stb128<kCpSc1>(c.ws, OFF_ZPART + ((c.g * TP + t) * D + 32 * c.r + rt * 16 + 4 * c.lq) * 4,
                     as_u32x4(v));
  }
}

// ---------------------------------------------------------------- kernel
__global__ void __launch_bounds__(NTH, 1) pi05_denoise_bs1(Params p) {
  extern __shared__ __attribute__((aligned(16))) float lds[];
  Ctx c;
  c.tid = threadIdx.x;
  c.lane = c.tid & 63;
  c.wave = c.tid >> 6;
  c.lr = c.lane & 15;
  c.lq = c.lane >> 4;
  c.g = blockIdx.x & 7;
  c.r = blockIdx.x >> 3;
  c.ws = make_rsrc(p.ws, WS_BYTES);
  c.kc = make_rsrc(p.kcache, (uint32_t)((size_t)p.NL * p.Lmax * HD * 2));
  c.vc = make_rsrc(p.vtcache, (uint32_t)((size_t)p.NL * p.Lmax * HD * 2));
  c.lds = lds;
  c.red = reinterpret_cast<f32x4*>(lds + L_RED);

  unsigned* err = reinterpret_cast<unsigned*>(p.ws + OFF_CTRL + 8);
  if (c.tid == 0 && xcc_id() != (unsigned)c.g) atomicOr(err, kErrXcd);
  Sync s;
  s.xline = reinterpret_cast<uint64_t*>(p.ws + OFF_XFLAG) + c.g * NR;
  s.gline = reinterpret_cast<uint64_t*>(p.ws + OFF_GFLAG);
  s.err = err;
  s.rank = c.r;
  s.xcd = c.g;
  s.nrank = NR;
  s.nxcd = NX;
  const uint64_t seq = ld_flag(reinterpret_cast<const uint64_t*>(p.ws + OFF_CTRL));
  s.e = seq << 32;

  // my two tokens' x_t into LDS
  if (c.tid < 64) {
    const int j = c.tid >> 5, a = c.tid & 31, t = c.r + 32 * j;
    lds[L_XT + j * AD + a] = t < p.Tv ? p.x_t[t * AD + a] : 0.f;
  }
  __syncthreads();

  const float dt = -1.0f / (float)p.S;
  uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  const int NL = p.NL;
#pragma unroll 1
  for (int step = 0; step < p.S; step++) {
#pragma unroll 1
    for (int l = 0; l < NL; l++) {
      const float* mod_in = p.mods + ((size_t)(step * NL + l) * 2 + 0) * 3 * D;
      const float* mod_post = p.mods + ((size_t)(step * NL + l) * 2 + 1) * 3 * D;
      if (l == 0) {
        stage_norm<0>(p, c, 0, nullptr, mod_in, mod_in + D);
      } else {
        const float* gprev = p.mods + ((size_t)(step * NL + l - 1) * 2 + 1) * 3 * D + 2 * D;
        stage_norm<1>(p, c, OFF_ZPART, gprev, mod_in, mod_in + D);
      }
      mark(p, c, 0, t0);
      {
        u32x4 w[2][8];
        sync_arrive(s);
        load_w_qkv(p, c, l, w);
        sync_wait_xcd(s);
        mark(p, c, 9, t0);
        stage_qkv(p, c, l, w);
      }
      mark(p, c, 1, t0);
      sync_arrive(s);
      sync_wait_xcd(s);
      mark(p, c, 9, t0);
      stage_att(p, c, l);
      mark(p, c, 2, t0);
      sync_arrive(s);
      sync_wait_xcd(s);
      mark(p, c, 9, t0);
      stage_comb(p, c);
      mark(p, c, 3, t0);
      {
        u32x4 w[2][2];
        sync_arrive(s);
        load_w_o(p, c, l, w);
        sync_wait_xcd(s);
        mark(p, c, 9, t0);
        stage_oproj(p, c, w);
      }
      mark(p, c, 4, t0);
      sync_arrive(s);
      sync_wait_grid(s);
      mark(p, c, 10, t0);
      stage_norm<1>(p, c, OFF_OPART, mod_in + 2 * D, mod_post, mod_post + D);
      mark(p, c, 5, t0);
      {
        u32x4 w[2][8];
        sync_arrive(s);
        load_w_gu(p, c, l, w);
        sync_wait_xcd(s);
        mark(p, c, 9, t0);
        stage_gu(p, c, w);
      }
      mark(p, c, 6, t0);
      {
        u32x4 w[2][4];
        sync_arrive(s);
        load_w_dn(p, c, l, w);
        sync_wait_xcd(s);
        mark(p, c, 9, t0);
        stage_dn(p, c, w);
      }
      mark(p, c, 7, t0);
      sync_arrive(s);
      sync_wait_grid(s);
      mark(p, c, 10, t0);
    }
    const float* gl = p.mods + ((size_t)(step * NL + NL - 1) * 2 + 1) * 3 * D + 2 * D;
    const float* mf = p.mod_final + (size_t)step * 3 * D;
    stage_norm<2>(p, c, OFF_ZPART, gl, mf, mf + D);
    stage_action(p, c, dt);
    mark(p, c, 8, t0);
  }
  if (c.g == 0 && c.tid < 64) {
    const int j = c.tid >> 5, a = c.tid & 31, t = c.r + 32 * j;
    if (t < p.Tv) p.x_t[t * AD + a] = lds[L_XT + j * AD + a];
  }
  if (blockIdx.x == 0 && c.tid == 0)
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p.ws + OFF_CTRL), seq + 1, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

__global__ void ws_zero(u32x4* p, size_t n16) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x)
    p[i] = u32x4{0, 0, 0, 0};
}

}  // namespace pi05
}  // namespace fa

// ================================================================= host C ABI
using namespace fa;

extern "C" size_t fa_pi05_workspace_bytes(int batch, int Tv, int Lmax) {
  (void)Tv;
  (void)Lmax;
  if (batch != 1) return 0;
  return pi05::WS_BYTES;
}

extern "C" int fa_pi05_max_batch(void) { return 1; }

extern "C" int fa_pi05_workspace_init(void* workspace, size_t bytes, fa_stream_t stream) {
  if (!workspace || bytes == 0 || (bytes & 15) || (reinterpret_cast<uintptr_t>(workspace) & 255))
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_workspace_init: workspace must be non-null, 256-byte aligned, "
                                          "size a non-zero multiple of 16");
  hipLaunchKernelGGL(pi05::ws_zero, dim3(1024), dim3(256), 0, (hipStream_t)stream, (u32x4*)workspace, bytes / 16);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return host::fail(FA_ERR_LAUNCH, "fa_pi05_workspace_init: %s", hipGetErrorString(e));
  return FA_OK;
}

extern "C" int fa_pi05_read_status(const void* workspace, unsigned* status) {
  if (!workspace || !status) return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_read_status: null argument");
  hipError_t e = hipMemcpy(status, static_cast<const unsigned char*>(workspace) + pi05::OFF_CTRL + 8, 4,
                           hipMemcpyDeviceToHost);
  if (e != hipSuccess) return host::fail(FA_ERR_LAUNCH, "fa_pi05_read_status: %s", hipGetErrorString(e));
  return FA_OK;
}

extern "C" int fa_pi05_denoise(const fa_pi05_args* a, fa_stream_t stream) {
  using namespace fa::pi05;
  if (!a) return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: args is NULL");
  if (a->weight_dtype != FA_DTYPE_BF16)
    return host::fail(FA_ERR_UNSUPPORTED, "fa_pi05_denoise: only bf16 weights are implemented (weight_dtype=%d)",
                      a->weight_dtype);
  if (a->s1 || a->so || a->s2 || a->s3)
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: fp8 row scales must be NULL for bf16 weights");
  if (a->srows != 0 || a->kvsrc_k || a->kvsrc_v)
    return host::fail(FA_ERR_UNSUPPORTED, "fa_pi05_denoise: the KV hand-off prologue (srows > 0) is not implemented");
  if (a->batch != 1)
    return host::fail(FA_ERR_UNSUPPORTED, "fa_pi05_denoise: batch=%d (this entry point runs batch 1)", a->batch);
  const void* ptrs[] = {a->w1, a->wo, a->w2, a->w3, a->mods, a->mod_final, a->rope_cos, a->rope_sin, a->w_ain,
                        a->b_ain, a->w_aout, a->b_aout, a->kcache, a->vtcache, a->x_t, a->workspace};
  const char* names[] = {"w1", "wo", "w2", "w3", "mods", "mod_final", "rope_cos", "rope_sin", "w_ain",
                         "b_ain", "w_aout", "b_aout", "kcache", "vtcache", "x_t", "workspace"};
  for (int i = 0; i < 16; i++) {
    if (!ptrs[i]) return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: %s is NULL", names[i]);
    if (reinterpret_cast<uintptr_t>(ptrs[i]) & 15)
      return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: %s is not 16-byte aligned", names[i]);
  }
  if (reinterpret_cast<uintptr_t>(a->workspace) & 255)
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: workspace is not 256-byte aligned");
  if (a->num_layers < 1 || a->num_steps < 1 || a->Tv < 1 || a->Tv > TP || a->Lp < 0)
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: need num_layers>=1, num_steps>=1, 1<=Tv<=%d, Lp>=0 "
                      "(got NL=%d S=%d Tv=%d Lp=%d)", TP, a->num_layers, a->num_steps, a->Tv, a->Lp);
  if (a->Lmax < a->Lp + a->Tv || (a->Lmax & 15))
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: Lmax=%d must be a multiple of 16 and >= Lp+Tv=%d",
                      a->Lmax, a->Lp + a->Tv);
  if (a->Lp + a->Tv > 8192)
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: Lp+Tv=%d exceeds 8192", a->Lp + a->Tv);
  if ((size_t)a->num_layers * a->Lmax * HD * 2 > 0x7fffffffu)
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: KV cache larger than 2 GiB per sample");
  if (a->xt_rows < a->Tv)
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: xt_rows=%d < Tv=%d", a->xt_rows, a->Tv);
  if (a->workspace_bytes < WS_BYTES)
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: workspace_bytes=%zu < required %u", a->workspace_bytes,
                      (unsigned)WS_BYTES);
  int rc = host::check_device((const void*)pi05_denoise_bs1, NTH, LDS_BYTES, NWG, "fa_pi05_denoise");
  if (rc != FA_OK) return rc;

  Params p;
  p.w1 = static_cast<const bf16*>(a->w1);
  p.wo = static_cast<const bf16*>(a->wo);
  p.w2 = static_cast<const bf16*>(a->w2);
  p.w3 = static_cast<const bf16*>(a->w3);
  p.mods = a->mods;
  p.mod_final = a->mod_final;
  p.rope_cos = a->rope_cos;
  p.rope_sin = a->rope_sin;
  p.w_ain = a->w_ain;
  p.b_ain = a->b_ain;
  p.w_aout = a->w_aout;
  p.b_aout = a->b_aout;
  p.kcache = static_cast<bf16*>(a->kcache);
  p.vtcache = static_cast<bf16*>(a->vtcache);
  p.x_t = a->x_t;
  p.stage_cycles = a->stage_cycles;
  p.ws = static_cast<unsigned char*>(a->workspace);
  p.NL = a->num_layers;
  p.Lp = a->Lp;
  p.Lmax = a->Lmax;
  p.S = a->num_steps;
  p.Tv = a->Tv;
  p.xt_rows = a->xt_rows;
  void* args[] = {&p};
  hipError_t e = hipLaunchCooperativeKernel((const void*)pi05_denoise_bs1, dim3(NWG), dim3(NTH), args, LDS_BYTES,
                                            (hipStream_t)stream);
  if (e != hipSuccess) return host::fail(FA_ERR_LAUNCH, "fa_pi05_denoise: cooperative launch failed: %s",
                                         hipGetErrorString(e));
  return FA_OK;
}
