// pi0.5 prefix prefill (the benchmark's prefill workload): the Gemma-2B-shaped backbone (D = 2048, 8 query heads /
// 1 K/V head of 256, F = 16384) over the Lp prefix tokens of each sample, in ONE cooperative launch
// of 256 workgroups x 8 waves on the stage engine (engine.h). Its product is the K/V cache the
// denoise loop reads: the QKV epilogue writes the RoPE'd keys into kcache rows [0, Lp) and the
// values into vtcache columns [0, Lp) of every layer, the layout the reference builds with
// compact_kv and the cache fill after its prefill (src/pi05/pack_weights.py:60-70;
// benchmarks/pi05/eval_numerics.py:50-57, 83-87).
//
// Per layer (grid barrier after each stage), token m = b * Lp + t of sample b:
//   N1   x = prefix hidden states (layer 0) or x += sum(down partials); xn = rms(x) (1 + w_in)
//   QKV  [M x 2560] = xn Wqkv^T; RoPE at position t; q -> fragment-ordered Q, k/v -> the caches
//   ATT  per (sample, 128-key chunk, 16 query tiles): every query row against the chunk's keys
//        (the prefix attends to itself without a mask), online softmax -> partial O + (m, l)
//   COMB combine of the key chunks -> attn [M x 2048]
//   O    [M x 2048] = attn Wo^T, K split 2 ways -> bf16 partials
// O, GU and DN read their token operand (attn, xn after N2, h) in MFMA fragment order.
//   N2   x += sum(partials); xn = rms(x) (1 + w_post), written in MFMA fragment order
//   GU   [M x 32768] = xn Wgu^T (gate/up rows interleaved, 512 x 128 tiles) -> h = gelu_tanh(g) u
//        [M x 16384], fragment order
//   DN   [M x 2048] = h Wdn^T (512 x 128 tiles), K split 8 ways -> bf16 partials
// The last layer stops after QKV: its attention and MLP outputs reach no cache entry.
// Two waves per SIMD (8 per workgroup): the tall MLP tiles keep the MFMA pipe busy about 1.4x as long
// as one wave per SIMD can, at a budget of 256 registers per lane in every stage.
#define FA_ENG_NWAVE 8
#include "engine.h"
#include "mqa256.h"
#include "../../include/flashact_mi355x.h"
#include "fa_host.h"

namespace fa {
namespace pf {
using namespace fa::eng;
using namespace fa::mqa;

constexpr int D = 2048, FF = 16384;
constexpr int QKVN = QD + 2 * HD;  // 2560 projection rows
constexpr int KS_O = 2, KS_DN = 8;  // K splits of the O and down projections
constexpr int MAX_TOKENS = 16384;  // batch x Lp
static_assert((size_t)NH * MAX_TOKENS < (1u << 20), "divmod_u: the combine rows stay below 2^20");

struct Layout {
  int B, Tv, M, MP, NQT, NKC;
  size_t x, xn, qf, attp, ml, attn, h, part, total;
};
// Tv = Lp: the stage templates of mqa256.h see the prefix tokens as the tokens of this launch.
__host__ __device__ inline Layout layout(int B, int Lp, int Lmax) {
  Layout L;
  L.B = B;
  L.Tv = Lp;
  L.M = B * Lp;
  L.MP = (L.M + 127) / 128 * 128;
  L.NQT = (NH * Lp + 15) / 16;
  L.NKC = (Lmax + KCH - 1) / KCH;
  size_t o = kWsDataBase;
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
  L.part = take((size_t)KS_DN * L.MP * D * 4);
  L.total = o;
  return L;
}
constexpr uint32_t OFF_CTRL = 0, OFF_FLAGS = 1024;

// Field names follow what the mqa256.h stages read: the cache offset Lp of those stages is 0 here
// (the prefix itself is written) and Tv is the prefix length.
struct Params {
  const bf16* wqkv;
  const bf16* wo;
  const bf16* wgu;
  const bf16* wdn;
  const float* ln_in;
  const float* ln_post;
  const float* rope_cos;
  const float* rope_sin;
  const float* x_in;  // [B][Tv][2048]
  bf16* kcache;       // [B][NL][Lmax][256]
  bf16* vtcache;      // [B][NL][256][Lmax]
  unsigned long long* stage_cycles;
  unsigned char* ws;
  Layout L;
  int NL, Lp, Lmax, Tv, B;
};

// h = gelu_tanh(g) u in MFMA fragment order (the down projection's tall-tile operand): rows 2f, 2f+1
// of the tile are gate f, up f; the lane's features f, f + 1 (f even) of token m are 4 bytes of the
// 16-byte slot (k-quarter (f % 32) / 8, token m % 16) of fragment (m / 16, f / 32).
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

// bf16 partial sums [split][MP][2048] of the down projection (tall tile, 8 bytes per lane and block).
// The next N1 reads all eight of them with the residual x: as fp32 they were 63 MB of the stage's
// 83 MB per layer at Lp = 968 (N1 and this stage's stores both bandwidth-bound). Each partial is
// rounded once to bf16 before the fp32 sum: the precision of the reference's bf16 backbone, whose
// residual stream itself is bf16; the range is fp32's.
struct EpiPartB {  // bf16 partial sums [split][MP][2048] of the down projection, rows staged whole
  static constexpr int kRowBytes = 8;
  static constexpr bool kStaged = true;
  rsrc_t ws;
  uint32_t off;
  int MP, split;
  __device__ u32x4 pack(int, f32x4 v) const { return u32x4{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), 0u, 0u}; }
  __device__ uint32_t row_off(int m, int n0) const { return off + (uint32_t)((((size_t)split * MP + m) * D + n0) * 2); }
};

struct EpiPart : NoPre {  // bf16 partial sums [split][MP][2048] of the O projection (as EpiPartB)
  static constexpr int kRowBytes = 8;
  static constexpr bool kStaged = true;
  rsrc_t ws;
  uint32_t off;
  int MP, split;
  __device__ u32x4 pack(int, f32x4 v) const { return u32x4{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), 0u, 0u}; }
  __device__ uint32_t row_off(int m, int n0) const { return off + (uint32_t)((((size_t)split * MP + m) * D + n0) * 2); }
};

// A token row per wave pair (q, q + 4) of a workgroup (q < 4): half hh = wave / 4 of the pair takes
// columns [1024 hh, 1024 hh + 1024), the lane columns 4 lane + 256 k + 1024 hh + i (k < 4), and the
// halves' sums of squares meet in LDS. (One row per wave left half the waves idle at Lp = 968 and
// needed two rounds of loads for eight down partials: N1 16.2 µs per layer.) Rows go pair-major,
// row m on workgroup m % 256, so they spread over every CU; every wave runs the same number of rounds,
// since the exchange is a workgroup barrier. FIRST: x = the prefix hidden states; otherwise x += the
// sum of the NS K-split partials (in split order; PB: bf16 partials, else fp32). Then xn = rms(x) (1 + w), with FRAG in MFMA fragment
// order (columns c..c+7 of token m, c % 8 = 0: the 16-byte slot (k-quarter (c % 32) / 8, token m % 16)
// of fragment (m / 16, c / 32)), else row-major [M][2048]. The QKV GEMM after N1 reads the row-major
// form: fragment slots written 16 bytes at a time by the waves of 16 different tokens took N1 from
// 10.0 to 12.8 µs per layer here, more than the fragment-order copies save in the GEMM.
template <bool FIRST, int NS, bool FRAG, bool PB = false>
__device__ __forceinline__ void stage_norm(const Params& p, rsrc_t ws, rsrc_t xin, const float* w) {
  static_assert(NWAVE == 8, "a row per wave pair");
  const Layout& L = p.L;
  const int lane = lane_id(), wv = wave_id(), q = wv & 3, hh = wv >> 2;
  float* red = reinterpret_cast<float*>(lds);  // [iteration parity][wave] sums of squares
  const int rounds = (L.M + NWG * 4 - 1) / (NWG * 4);
#pragma unroll 1
  for (int it = 0; it < rounds; it++) {
    const int m = (it * 4 + q) * NWG + vwg();
    const bool has = m < L.M;
    const int mr = has ? m : 0;  // a pair without a row reads row 0 and stores nothing
    f32x4 x[4];
    if (FIRST) {
#pragma unroll
      for (int k = 0; k < 4; k++)
        x[k] = as_f32x4(ldb128<kCpPlain>(xin, (uint32_t)(((size_t)mr * D + 4 * lane + 256 * k + 1024 * hh) * 4)));
    } else {
      u32x4 xo[4];
      f32x4 pf[NS][4];
      if constexpr (PB) {
        u32x2 pr[NS][4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const int d = 4 * lane + 256 * k + 1024 * hh;
          xo[k] = ldb128<kCpSc1>(ws, (uint32_t)(L.x + ((size_t)mr * D + d) * 4));
#pragma unroll
          for (int s = 0; s < NS; s++)
            pr[s][k] = ldb64<kCpSc1>(ws, (uint32_t)(L.part + (((size_t)s * L.MP + mr) * D + d) * 2));
        }
#pragma unroll
        for (int s = 0; s < NS; s++)
#pragma unroll
          for (int k = 0; k < 4; k++)
            pf[s][k] = f32x4{bf_lo(pr[s][k][0]), bf_hi(pr[s][k][0]), bf_lo(pr[s][k][1]), bf_hi(pr[s][k][1])};
      } else {
        u32x4 pr[NS][4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
          const int d = 4 * lane + 256 * k + 1024 * hh;
          xo[k] = ldb128<kCpSc1>(ws, (uint32_t)(L.x + ((size_t)mr * D + d) * 4));
#pragma unroll
          for (int s = 0; s < NS; s++)
            pr[s][k] = ldb128<kCpSc1>(ws, (uint32_t)(L.part + (((size_t)s * L.MP + mr) * D + d) * 4));
        }
#pragma unroll
        for (int s = 0; s < NS; s++)
#pragma unroll
          for (int k = 0; k < 4; k++) pf[s][k] = as_f32x4(pr[s][k]);
      }
#pragma unroll
      for (int k = 0; k < 4; k++) {
        f32x4 t = pf[0][k];
#pragma unroll
        for (int sp = 1; sp < NS; sp++) t += pf[sp][k];
        x[k] = as_f32x4(xo[k]) + t;
      }
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < 4; k++) ss += x[k][0] * x[k][0] + x[k][1] * x[k][1] + x[k][2] * x[k][2] + x[k][3] * x[k][3];
    ss = wave_sum(ss);
    if (lane == 0) red[(it & 1) * NWAVE + wv] = ss;
    __syncthreads();
    const float rr = rsqrtf((red[(it & 1) * NWAVE + q] + red[(it & 1) * NWAVE + q + 4]) / (float)D + 1e-6f);
    if (!has) continue;
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int d = 4 * lane + 256 * k + 1024 * hh;
      const f32x4 wv4 = *reinterpret_cast<const f32x4*>(w + d);
      f32x4 h;
#pragma unroll
      for (int i = 0; i < 4; i++) h[i] = x[k][i] * rr * (1.0f + wv4[i]);
      st_b128(ws, (uint32_t)(L.x + ((size_t)m * D + d) * 4), as_u32x4(x[k]));
      const unsigned lo = pack_bf16x2(h[0], h[1]), hi = pack_bf16x2(h[2], h[3]);
      if (!FRAG) {
        st_b64(ws, (uint32_t)(L.xn + ((size_t)m * D + d) * 2), u32x2{lo, hi});
        continue;
      }
      // 16-byte fragment slots: lanes (2j, 2j + 1) hold columns 8j .. 8j + 7 of this k; the even lane
      // stores the slot for even k, the odd lane for odd k
      const unsigned plo = swap_adj(lo), phi = swap_adj(hi);
      if ((lane & 1) == (k & 1)) {
        const int c = d & ~7;
        const uint32_t xa = (uint32_t)((((size_t)(m >> 4) * (D / 32) + (c >> 5)) * 64 + ((c & 31) >> 3) * 16 + (m & 15)) * 16);
        st_b128(ws, (uint32_t)L.xn + xa, (lane & 1) ? u32x4{plo, phi, lo, hi} : u32x4{lo, hi, plo, phi});
      }
    }
  }
}

constexpr uint32_t LDS_GEMM = GemmShape<4, 4>::LDS > TALL_LDS ? GemmShape<4, 4>::LDS : TALL_LDS;
constexpr uint32_t LDS_ATTG = LDS_GEMM > ATT_LDS ? LDS_GEMM : ATT_LDS;
constexpr uint32_t LDS_STAGE = staged_d_lds<NWAVE, 4>();  // the down projection's staged rows
constexpr uint32_t LDS_BYTES = LDS_ATTG > LDS_STAGE ? LDS_ATTG : LDS_STAGE;
static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");

__device__ __forceinline__ void mark(const Params& p, int idx, uint64_t& t0) {
  if (p.stage_cycles) {  // t0 moves in every wave: a value set under the thread test would live in VGPRs
    const uint64_t t1 = __builtin_amdgcn_s_memrealtime();
    if (grid_thread0()) p.stage_cycles[idx] += t1 - t0;
    t0 = t1;
  }
}

__global__ void __launch_bounds__(NTHR, 1) prefill_kernel(Params p) {
  const Layout& L = p.L;
  const rsrc_t ws = rsrc_all(p.ws);
  const rsrc_t kc = rsrc_all(p.kcache);
  const rsrc_t vc = rsrc_all(p.vtcache);
  const rsrc_t xin = rsrc_all(p.x_in);
  Grid grid;
  grid.flags = reinterpret_cast<uint64_t*>(p.ws + OFF_FLAGS);
  grid.err = reinterpret_cast<unsigned*>(p.ws + OFF_CTRL + 8);
  // every lane loaded the same word: its halves go to SGPRs, and so do the barrier epochs after it
  const uint64_t seq_v = ld_flag(reinterpret_cast<const uint64_t*>(p.ws + OFF_CTRL));
  const uint64_t seq = (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(seq_v >> 32)) << 32 |
                       (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)seq_v);
  grid.e = seq << 32;
  if (xcc_id() != (blockIdx.x & 7u) && tid() == 0) atomicOr(grid.err, kErrXcd);
  if (grid_thread0())
    __hip_atomic_store(reinterpret_cast<unsigned*>(p.ws + kWsOwner), kOwnerPrefill, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  const int NL = p.NL;
  const float rtv = rcp_u(p.Tv);
  uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  const uint32_t mb16 = (uint32_t)((L.M + 15) / 16 * 16);  // tokens of the fragment-ordered operands
  GemmArgsF gxf{make_rsrc(p.ws + L.xn, mb16 * D * 2), nullptr, D / 32, D, L.M};
  GemmArgs gx{reinterpret_cast<const bf16*>(p.ws + L.xn), nullptr, D, D, L.M};
  GemmArgs ga{reinterpret_cast<const bf16*>(p.ws + L.attn), nullptr, QD, QD, L.M};
  GemmArgsF ghf{make_rsrc(p.ws + L.h, mb16 * FF * 2), nullptr, FF / 32, FF, L.M};
#pragma unroll 1
  for (int l = 0; l < NL; l++) {
    if (l == 0)
      stage_norm<true, 1, false>(p, ws, xin, p.ln_in);
    else
      stage_norm<false, KS_DN, false, true>(p, ws, xin, p.ln_in + (size_t)l * D);
    mark(p, 0, t0);
    grid_sync(grid);
    mark(p, 9, t0);
    {
      EpiQKV e{ws, kc, vc, p.rope_cos, p.rope_sin, (uint32_t)L.qf, L.NQT, p.Tv, NL, p.Lmax, p.Lp, l, 0, rtv};
      gx.W = p.wqkv + (size_t)l * QKVN * D;
      gemm_stage<3, 4>(gx, QKVN, D, 1, e);  // 96-token tiles: 220 items (160 of 128): QKV 29.1 -> 26.3 us per layer
    }
    mark(p, 1, t0);
    if (l == NL - 1) break;  // the last layer's K/V are in the caches
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
      gemm_stage<4, 4, true>(ga, D, QD, KS_O, e);
    }
    mark(p, 4, t0);
    grid_sync(grid);
    mark(p, 9, t0);
    stage_norm<false, KS_O, true, true>(p, ws, xin, p.ln_post + (size_t)l * D);
    mark(p, 5, t0);
    grid_sync(grid);
    mark(p, 9, t0);
    {
      EpiGeluF e{ws, (uint32_t)L.h, 0};
      gxf.W = p.wgu + (size_t)l * 2 * FF * D;
      gemm_stage_tall(gxf, 2 * FF, D, 1, e);
    }
    mark(p, 6, t0);
    grid_sync(grid);
    mark(p, 9, t0);
    {
      EpiPartB e{ws, (uint32_t)L.part, L.MP, 0};
      ghf.W = p.wdn + (size_t)l * D * FF;
      gemm_stage_tall(ghf, D, FF, KS_DN, e);
    }
    mark(p, 7, t0);
    grid_sync(grid);
    mark(p, 9, t0);
  }
  if (grid_thread0())
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p.ws + OFF_CTRL), seq + 1, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace pf
}  // namespace fa

// ================================================================= host C ABI
using namespace fa;

extern "C" size_t fa_pi05_prefill_workspace_bytes(int batch, int Lp, int Lmax) {
  if (batch < 1 || Lp < 1 || Lmax < Lp || (size_t)batch * Lp > (size_t)pf::MAX_TOKENS) return 0;
  const size_t n = pf::layout(batch, Lp, Lmax).total;
  return n < 0xffffffffull ? n : 0;
}

extern "C" int fa_pi05_prefill(const fa_prefill_args* a, fa_stream_t stream) {
  using namespace fa::pf;
  if (!a) return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_prefill: args is NULL");
  if (a->weight_dtype != FA_DTYPE_BF16)
    return host::fail(FA_ERR_UNSUPPORTED, "fa_pi05_prefill: only bf16 weights are implemented (weight_dtype=%d)",
                      a->weight_dtype);
  const void* ptrs[] = {a->wqkv, a->wo, a->wgu, a->wdn, a->ln_in, a->ln_post, a->rope_cos, a->rope_sin,
                        a->x, a->kcache, a->vtcache, a->workspace};
  const char* names[] = {"wqkv", "wo", "wgu", "wdn", "ln_in", "ln_post", "rope_cos", "rope_sin",
                         "x", "kcache", "vtcache", "workspace"};
  for (int i = 0; i < 12; i++) {
    if (!ptrs[i]) return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_prefill: %s is NULL", names[i]);
    if (reinterpret_cast<uintptr_t>(ptrs[i]) & 15)
      return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_prefill: %s is not 16-byte aligned", names[i]);
  }
  if (reinterpret_cast<uintptr_t>(a->workspace) & 255)
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_prefill: workspace is not 256-byte aligned");
  if (a->num_layers < 1 || a->Lp < 1 || a->batch < 1)
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_prefill: need num_layers>=1, Lp>=1, batch>=1 (got NL=%d Lp=%d "
                      "batch=%d)", a->num_layers, a->Lp, a->batch);
  if (a->Lmax < a->Lp || (a->Lmax & 15))
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_prefill: Lmax=%d must be a multiple of 16 and >= Lp=%d", a->Lmax,
                      a->Lp);
  if ((size_t)a->batch * a->Lp > (size_t)MAX_TOKENS)
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_prefill: batch x Lp = %d exceeds %d tokens", a->batch * a->Lp,
                      MAX_TOKENS);
  const size_t cache_bytes = (size_t)a->batch * a->num_layers * a->Lmax * HD * 2;
  if (cache_bytes >= 0xffffffffull)
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_prefill: caches of %zu bytes exceed the 4 GB buffer range",
                      cache_bytes);
  if ((size_t)a->batch * a->Lp * D * 4 >= 0xffffffffull)
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_prefill: x exceeds the 4 GB buffer range");
  const size_t need = fa_pi05_prefill_workspace_bytes(a->batch, a->Lp, a->Lmax);
  if (need == 0 || a->workspace_bytes < need)
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_prefill: workspace_bytes=%zu < required %zu", a->workspace_bytes,
                      need);
  int rc = host::check_device((const void*)prefill_kernel, NTHR, LDS_BYTES, NWG, "fa_pi05_prefill");
  if (rc != FA_OK) return rc;
  Params p;
  p.wqkv = static_cast<const bf16*>(a->wqkv);
  p.wo = static_cast<const bf16*>(a->wo);
  p.wgu = static_cast<const bf16*>(a->wgu);
  p.wdn = static_cast<const bf16*>(a->wdn);
  p.ln_in = a->ln_in;
  p.ln_post = a->ln_post;
  p.rope_cos = a->rope_cos;
  p.rope_sin = a->rope_sin;
  p.x_in = a->x;
  p.kcache = static_cast<bf16*>(a->kcache);
  p.vtcache = static_cast<bf16*>(a->vtcache);
  p.stage_cycles = a->stage_cycles;
  p.ws = static_cast<unsigned char*>(a->workspace);
  p.L = layout(a->batch, a->Lp, a->Lmax);
  p.NL = a->num_layers;
  p.Lp = 0;  // cache rows written from 0: the prefix itself
  p.Lmax = a->Lmax;
  p.Tv = a->Lp;
  p.B = a->batch;
  void* args[] = {&p};
  return host::coop_launch((const void*)prefill_kernel, NWG, NTHR, args, LDS_BYTES, stream, "fa_pi05_prefill");
}
