// pi0.5 action-expert denoise loop for a batch of samples (the batch-16 workload: batch 16, M = 800
// action tokens per GEMM): the whole S-step Euler loop in ONE cooperative launch of 256
// workgroups x 4 waves, built on the stage engine (engine.h). This is the MFMA-bound regime, so
// the GEMMs are 128-token tiles over all samples at once.
//
// Per layer (grid barrier after each stage), token m = b * Tv + t of sample b:
//   N1   x = embed(x_t) (layer 0) or x += gate_post * sum(down partials); xn = adaRMS(x)
//   QKV  [M x 2560] = xn W1^T (96-token tiles); RoPE; q -> per-sample fragment-ordered Q; k, v -> the caller's
//        caches (row / column Lp + t of layer l), as the reference does (src/pi05/mk6.cu:307-310)
//   ATT  per (sample, 128-key chunk, group of 16 query tiles): MQA over the chunk (8 heads x Tv
//        query rows share the one K/V head), online softmax, normalised partial O + (m, l)
//   COMB flash-decoding combine of the key chunks -> attn [M x 2048]
//   O    [M x 1024] = attn Wo^T, K split 4 ways -> fp32 partials
//   N2   x += gate_in * sum(partials); xn = adaRMS(x)
//   GU   [M x 8192] = xn W2^T (gate/up rows interleaved; 256 x 128 tall tiles) -> h = gelu_tanh(g) u
//        [M x 4096]
//   DN   [M x 1024] = h W3^T, K split 4 ways -> fp32 partials
// (GEMMs other than GU: 128-row weight tiles of 128 tokens, 96 for QKV, in engine.h gemm_tile.) Every
// GEMM reads its token operand (xn, attn, h) in MFMA fragment order.
// then the final norm, action projection and Euler update (src/pi05/mk6.cu:502-517).
#include "engine.h"
#include "mqa256.h"
#include "../../include/flashact_mi355x.h"
#include "fa_host.h"

namespace fa {
namespace pb {
using namespace fa::eng;
using namespace fa::mqa;

constexpr int D = 1024, AD = 32, FF = 4096;
constexpr int KSPLIT = 4;    // K split of the O and down projections
constexpr int MAX_TOKENS = 4096;
static_assert((size_t)NH * MAX_TOKENS < (1u << 20), "divmod_u: the combine rows stay below 2^20");

// Workspace layout (bytes), a function of (B, Tv, Lmax).
struct Layout {
  int B, Tv, M, MP, NQT, NKC;
  size_t x, xn, qf, attp, ml, attn, h, part, total;
};
__host__ __device__ inline Layout layout(int B, int Tv, int Lmax) {
  Layout L;
  L.B = B;
  L.Tv = Tv;
  L.M = B * Tv;
  L.MP = (L.M + 127) / 128 * 128;
  L.NQT = (NH * Tv + 15) / 16;
  L.NKC = (Lmax + KCH - 1) / KCH;
  size_t o = kWsDataBase;  // control words, epoch flags and counters below
  auto take = [&](size_t n) {
    const size_t r = o;
    o += (n + 255) / 256 * 256;
    return r;
  };
  L.x = take((size_t)L.MP * D * 4);
  L.xn = take((size_t)L.MP * D * 2);
  L.qf = take((size_t)B * L.NQT * 16 * HD * 2);
  L.attp = take((size_t)B * L.NKC * L.NQT * 16 * HD * 2);
  L.ml = take((size_t)B * L.NKC * L.NQT * 16 * 8);
  L.attn = take((size_t)L.MP * QD * 2);
  L.h = take((size_t)L.MP * FF * 2);
  L.part = take((size_t)KSPLIT * L.MP * D * 4);
  L.total = o;
  return L;
}
constexpr uint32_t OFF_CTRL = 0, OFF_FLAGS = 1024;

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
  bf16* kcache;  // [B][NL][Lmax][256]
  bf16* vtcache; // [B][NL][256][Lmax]
  float* x_t;    // [B][xt_rows][32]
  unsigned long long* stage_cycles;
  unsigned char* ws;
  Layout L;
  int NL, Lp, Lmax, S, Tv, B, xt_rows;
};

// Gate/up epilogue: rows 2f, 2f+1 of the tile are gate f, up f -> h = gelu_tanh(g) u in MFMA fragment
// order (the down projection's token operand): the lane's features f, f + 1 (f even) of token m are
// 4 bytes of the 16-byte slot (k-quarter (f % 32) / 8, token m % 16) of fragment (m / 16, f / 32).
struct EpiGeluF {
  rsrc_t ws;
  uint32_t off;
  int split;
  __device__ void operator()(int n, int m, f32x4 v) const {
    const int f = n >> 1;
    const uint32_t o = off + (uint32_t)(((((size_t)(m >> 4) * (FF / 32) + (f >> 5)) * 64 + ((f & 31) >> 3) * 16 +
                                          (m & 15)) * 16) + (f & 7) * 2);
    st_b32(ws, o, pack_bf16x2(gelu_tanh(v[0]) * v[1], gelu_tanh(v[2]) * v[3]));
  }
};

struct EpiPart : NoPre {  // fp32 partial sums [split][MP][1024]
  static constexpr int kRowBytes = 16;
  static constexpr bool kStaged = false;
  rsrc_t ws;
  uint32_t off;
  int MP, split;
  __device__ u32x4 pack(int, f32x4 v) const { return as_u32x4(v); }
  __device__ uint32_t row_off(int m, int n0) const { return off + (uint32_t)((((size_t)split * MP + m) * D + n0) * 4); }
};

// ---------------------------------------------------------------- norm rows
// One wave per token row; lane holds columns 4 lane + 256 k + i. MODE 0: x = embed(x_t);
// MODE 1: x += gate * sum of the K-split partials; MODE 2: as 1, then final norm + action
// projection + Euler update of x_t. xn is stored in MFMA fragment order (column d of token m: 8 bytes
// of the slot (k-quarter (d % 32) / 8, token m % 16) of fragment (m / 16, d / 32)).
template <int MODE>
__device__ __forceinline__ void stage_norm(const Params& p, rsrc_t ws, rsrc_t xtr, const float* gate, const float* scale, const float* shift,
                           float dt) {
  const Layout& L = p.L;
  const int lane = lane_id();
  const int nwave = NWG * 4;
  // wave-uniform descriptors with 32-bit lane offsets (per-lane 64-bit pointers cost two VGPRs each,
  // which the compiler kept live across the layer loop and spilled)
  const rsrc_t rg = make_rsrc(gate, gate ? D * 4 : 0), rsc = make_rsrc(scale, D * 4), rsh = make_rsrc(shift, D * 4);
  const rsrc_t rbi = make_rsrc(p.b_ain, D * 4), rwi = make_rsrc(p.w_ain, D * AD * 4);
  const rsrc_t rwo = make_rsrc(p.w_aout, AD * D * 4), rbo = make_rsrc(p.b_aout, AD * 4);
#pragma unroll 1
  for (int m = wave_id() * NWG + (int)blockIdx.x; m < L.M; m += nwave) {
    const int b = m / p.Tv, t = m - b * p.Tv;
    const uint32_t xto = (uint32_t)(((size_t)b * p.xt_rows + t) * AD * 4);
    f32x4 x[4];
    if (MODE == 0) {
      const float xl = lane < AD ? ldbf32<kCpSc1>(xtr, xto + lane * 4) : 0.f;
      float xa[AD];
#pragma unroll
      for (int a = 0; a < AD; a++) xa[a] = __shfl(xl, a, 64);
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int d = 4 * lane + 256 * k;
        const f32x4 bb = as_f32x4(ldb128<kCpPlain>(rbi, d * 4));
#pragma unroll
        for (int i = 0; i < 4; i++) {
          float s = bb[i];
#pragma unroll
          for (int q = 0; q < 8; q++) {
            const f32x4 wv = as_f32x4(ldb128<kCpPlain>(rwi, ((d + i) * AD + 4 * q) * 4));
#pragma unroll
            for (int e = 0; e < 4; e++) s = fmaf(wv[e], xa[4 * q + e], s);
          }
          x[k][i] = s;
        }
      }
    } else {
      u32x4 pr[KSPLIT][4], xo[4];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int d = 4 * lane + 256 * k;
        xo[k] = ldb128<kCpSc1>(ws, (uint32_t)(L.x + ((size_t)m * D + d) * 4));
#pragma unroll
        for (int s = 0; s < KSPLIT; s++)
          pr[s][k] = ldb128<kCpSc1>(ws, (uint32_t)(L.part + (((size_t)s * L.MP + m) * D + d) * 4));
      }
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int d = 4 * lane + 256 * k;
        f32x4 s = as_f32x4(pr[0][k]);
#pragma unroll
        for (int sp = 1; sp < KSPLIT; sp++) s += as_f32x4(pr[sp][k]);
        const f32x4 gt = as_f32x4(ldb128<kCpPlain>(rg, d * 4));
        x[k] = as_f32x4(xo[k]) + gt * s;
      }
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) ss += x[k][0] * x[k][0] + x[k][1] * x[k][1] + x[k][2] * x[k][2] + x[k][3] * x[k][3];
    const float rr = rsqrtf(wave_sum(ss) / (float)D + 1e-6f);
    f32x4 h[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int d = 4 * lane + 256 * k;
      const f32x4 sc = as_f32x4(ldb128<kCpPlain>(rsc, d * 4));
      const f32x4 sh = as_f32x4(ldb128<kCpPlain>(rsh, d * 4));
#pragma unroll
      for (int i = 0; i < 4; i++) h[k][i] = x[k][i] * rr * (1.0f + sc[i]) + sh[i];
    }
    if (MODE != 2) {
#pragma unroll
      for (int k = 0; k < 4; k++) {
        const int d = 4 * lane + 256 * k;
        st_b128(ws, (uint32_t)(L.x + ((size_t)m * D + d) * 4), as_u32x4(x[k]));
        // 16-byte fragment slots: lanes (2j, 2j + 1) hold columns 8j .. 8j + 7 of this k; the even
        // lane stores the slot for even k, the odd lane for odd k
        const unsigned lo = pack_bf16x2(h[k][0], h[k][1]), hi = pack_bf16x2(h[k][2], h[k][3]);
        const unsigned plo = swap_adj(lo), phi = swap_adj(hi);
        if ((lane & 1) == (k & 1)) {
          const int c = d & ~7;
          const uint32_t xa = (uint32_t)((((size_t)(m >> 4) * (D / 32) + (c >> 5)) * 64 + ((c & 31) >> 3) * 16 + (m & 15)) * 16);
          st_b128(ws, (uint32_t)L.xn + xa, (lane & 1) ? u32x4{plo, phi, lo, hi} : u32x4{lo, hi, plo, phi});
        }
      }
    } else {
      float acc = 0.f;  // lane a < 32 ends with v[a]
#pragma unroll 1
      for (int a0 = 0; a0 < AD; a0 += 8) {
        f32x4 wv[8][4];
#pragma unroll
        for (int a = 0; a < 8; a++)
#pragma unroll
          for (int k = 0; k < 4; k++)
            wv[a][k] = as_f32x4(ldb128<kCpPlain>(rwo, ((a0 + a) * D + 4 * lane + 256 * k) * 4));
#pragma unroll
        for (int a = 0; a < 8; a++) {
          float s = 0.f;
#pragma unroll
          for (int k = 0; k < 4; k++)
            s += wv[a][k][0] * h[k][0] + wv[a][k][1] * h[k][1] + wv[a][k][2] * h[k][2] + wv[a][k][3] * h[k][3];
          s = wave_sum(s);
          if (lane == a0 + a) acc = s;
        }
      }
      if (lane < AD) {
        const float xo = ldbf32<kCpSc1>(xtr, xto + lane * 4);
        __builtin_amdgcn_raw_buffer_store_b32(as_u32(xo + dt * (acc + ldbf32<kCpPlain>(rbo, lane * 4))), xtr, xto + lane * 4,
                                              0, kCpSc1);
      }
    }
  }
}

// ---------------------------------------------------------------- the kernel
constexpr uint32_t LDS_GEMM = GemmShape<4, 4>::LDS > TALL_LDS ? GemmShape<4, 4>::LDS : TALL_LDS;
constexpr uint32_t LDS_BYTES = LDS_GEMM > ATT_LDS ? LDS_GEMM : ATT_LDS;
static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");

__device__ __forceinline__ void mark(const Params& p, int idx, uint64_t& t0) {
  if (p.stage_cycles && blockIdx.x == 0 && threadIdx.x == 0) {
    const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
    p.stage_cycles[idx] += t1 - t0;
    t0 = t1;
  }
}

__global__ void __launch_bounds__(NTHR, 1) pi05_batched_kernel(Params p) {
  const Layout& L = p.L;
  const rsrc_t ws = rsrc_all(p.ws);
  const rsrc_t kc = rsrc_all(p.kcache);
  const rsrc_t vc = rsrc_all(p.vtcache);
  const rsrc_t xtr = make_rsrc(p.x_t, (uint32_t)((size_t)p.B * p.xt_rows * AD * 4));
  Grid grid;
  grid.flags = reinterpret_cast<uint64_t*>(p.ws + OFF_FLAGS);
  grid.err = reinterpret_cast<unsigned*>(p.ws + OFF_CTRL + 8);
  const uint64_t seq = ld_flag(reinterpret_cast<const uint64_t*>(p.ws + OFF_CTRL));
  grid.e = seq << 32;
  if (threadIdx.x == 0 && xcc_id() != (blockIdx.x & 7u)) atomicOr(grid.err, kErrXcd);
  if (blockIdx.x == 0 && threadIdx.x == 0)
    __hip_atomic_store(reinterpret_cast<unsigned*>(p.ws + kWsOwner), kOwnerPi05Batched, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  const int NL = p.NL;
  const float rtv = rcp_u(p.Tv);
  const float dt = -1.0f / (float)p.S;
  uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  const uint32_t mb16 = (uint32_t)((L.M + 15) / 16 * 16);  // tokens of the fragment-ordered operands
  GemmArgsF gxf{make_rsrc(p.ws + L.xn, mb16 * D * 2), nullptr, D / 32, D, L.M};
  GemmArgs gx{reinterpret_cast<const bf16*>(p.ws + L.xn), nullptr, D, D, L.M};
  GemmArgs ga{reinterpret_cast<const bf16*>(p.ws + L.attn), nullptr, QD, QD, L.M};
  GemmArgs gh{reinterpret_cast<const bf16*>(p.ws + L.h), nullptr, FF, FF, L.M};
#pragma unroll 1
  for (int step = 0; step < p.S; step++) {
#pragma unroll 1
    for (int l = 0; l < NL; l++) {
      const int li = step * NL + l;
      const float* mod_in = p.mods + ((size_t)li * 2 + 0) * 3 * D;
      const float* mod_post = p.mods + ((size_t)li * 2 + 1) * 3 * D;
      if (l == 0)
        stage_norm<0>(p, ws, xtr, nullptr, mod_in, mod_in + D, 0.f);
      else
        stage_norm<1>(p, ws, xtr, mod_post - 6 * D + 2 * D, mod_in, mod_in + D, 0.f);
      mark(p, 0, t0);
      grid_sync(grid);
      mark(p, 9, t0);
      {
        EpiQKV e{ws, kc, vc, p.rope_cos, p.rope_sin, (uint32_t)L.qf, L.NQT, p.Tv, NL, p.Lmax, p.Lp, l, 0, rtv};
        gx.W = p.w1 + (size_t)l * 2560 * D;
        gemm_stage<3, 4, true>(gx, 2560, D, 1, e);  // 96-token tiles: 180 items fill more of the 256 CUs than 140
      }
      mark(p, 1, t0);
      grid_sync(grid);
      mark(p, 9, t0);
      stage_att(p, ws, l);
      mark(p, 2, t0);
      grid_sync(grid);
      mark(p, 9, t0);
      stage_comb(p, ws);
      mark(p, 3, t0);
      grid_sync(grid);
      mark(p, 9, t0);
      {
        EpiPart e{{}, ws, (uint32_t)L.part, L.MP, 0};
        ga.W = p.wo + (size_t)l * D * QD;
        gemm_stage<4, 4, true, 2, true>(ga, D, QD, KSPLIT, e);
      }
      mark(p, 4, t0);
      grid_sync(grid);
      mark(p, 9, t0);
      stage_norm<1>(p, ws, xtr, mod_in + 2 * D, mod_post, mod_post + D, 0.f);
      mark(p, 5, t0);
      grid_sync(grid);
      mark(p, 9, t0);
      {
        EpiGeluF e{ws, (uint32_t)L.h, 0};
        gxf.W = p.w2 + (size_t)l * 8192 * D;
        gemm_stage_tall(gxf, 8192, D, 1, e);
      }
      mark(p, 6, t0);
      grid_sync(grid);
      mark(p, 9, t0);
      {
        EpiPart e{{}, ws, (uint32_t)L.part, L.MP, 0};
        gh.W = p.w3 + (size_t)l * D * FF;
        gemm_stage<4, 4, true, 2, true>(gh, D, FF, KSPLIT, e);
      }
      mark(p, 7, t0);
      grid_sync(grid);
      mark(p, 9, t0);
    }
    const int li = step * NL + NL - 1;
    const float* gl = p.mods + ((size_t)li * 2 + 1) * 3 * D + 2 * D;
    const float* mf = p.mod_final + (size_t)step * 3 * D;
    stage_norm<2>(p, ws, xtr, gl, mf, mf + D, dt);
    mark(p, 8, t0);
    grid_sync(grid);  // x_t of every token is final before the next step's embed reads it
    mark(p, 9, t0);
  }
  if (blockIdx.x == 0 && threadIdx.x == 0)
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p.ws + OFF_CTRL), seq + 1, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace pb
}  // namespace fa

// ================================================================= host side
namespace fa {

// Batched launch of fa_pi05_denoise (batch >= 2); argument checks common to both paths are done
// by the caller in pi05_bs1.hip.
size_t pi05_batched_workspace_bytes(int batch, int Tv, int Lmax) {
  if (batch < 1 || Tv < 1 || Lmax < 16) return 0;
  if ((size_t)batch * Tv > (size_t)pb::MAX_TOKENS) return 0;
  const size_t n = pb::layout(batch, Tv, Lmax).total;
  return n < 0xffffffffull ? n : 0;
}

int pi05_denoise_batched(const fa_pi05_args* a, fa_stream_t stream) {
  using namespace fa::pb;
  if ((size_t)a->batch * a->Tv > (size_t)MAX_TOKENS)
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: batch x Tv = %d exceeds %d tokens", a->batch * a->Tv,
                      MAX_TOKENS);
  const size_t need = pi05_batched_workspace_bytes(a->batch, a->Tv, a->Lmax);
  if (need == 0 || a->workspace_bytes < need)
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: workspace of %zu bytes, batch %d needs %zu",
                      a->workspace_bytes, a->batch, need);
  const size_t cache_bytes = (size_t)a->batch * a->num_layers * a->Lmax * HD * 2;
  if (cache_bytes >= 0xffffffffull)
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: caches of %zu bytes exceed the 4 GB buffer range",
                      cache_bytes);
  if (a->trace)
    return host::fail(FA_ERR_UNSUPPORTED, "fa_pi05_denoise: per-wave traces exist for batch 1 only");
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
  p.L = layout(a->batch, a->Tv, a->Lmax);
  p.NL = a->num_layers;
  p.Lp = a->Lp;
  p.Lmax = a->Lmax;
  p.S = a->num_steps;
  p.Tv = a->Tv;
  p.B = a->batch;
  p.xt_rows = a->xt_rows;
  int rc = host::check_device((const void*)pb::pi05_batched_kernel, NTHR, LDS_BYTES, NWG, "fa_pi05_denoise");
  if (rc != FA_OK) return rc;
  if (a->srows > 0 && (rc = pi05_kv_handoff(a, stream)) != FA_OK) return rc;
  void* args[] = {&p};
  return host::coop_launch((const void*)pb::pi05_batched_kernel, NWG, NTHR, args, LDS_BYTES, stream,
                           "fa_pi05_denoise (batched)");
}

}  // namespace fa
