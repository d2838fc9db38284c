// pi0.5 action-expert denoise loop, batch 1: the whole S-step Euler loop in ONE cooperative
// launch of 256 workgroups (one per CU) on gfx950. Each workgroup runs 6 waves:
//   waves 0-3  compute waves. Each is an independent agent: it owns token tile w (tokens
//              16w..16w+15) in every GEMM and attention stage and signals its own barrier flag,
//              so no workgroup barrier is executed after the prologue.
//   waves 4-5  loader waves. They stream this CU's share of every layer's weights, plus the
//              first 32 prefix keys/values of its attention chunk, HBM -> LDS ring with
//              global_load_lds_dwordx4, free-running ahead of the compute waves.
//
// Work decomposition (XCD-aware; XCD g = blockIdx % 8, rank r = blockIdx / 8 in 0..31):
//   XCD g owns query head g, the MLP columns f in [512g, 512g+512) and the K-windows g of the
//   O and down projections. Per layer (sync after each stage in brackets):
//     N1 [X] QKV [X] ATT [X] COMB [X] O {exchange} N2 [X] GU [X] DN {exchange}
//   [X] = XCD sync point: every compute wave of the XCD stores its epoch to its own flag slot. Before
//         ATT (whose waves read q and this step's keys from every QKV rank) each wave polls the
//         XCD's 128 slots; before QKV, COMB, O, GU and DN each wave polls only the waves that wrote
//         its operands (COMB: the 8 attention ranks of its chunks; DN: one group of 16 gate/up ranks
//         per 8-k-step chunk of its K loop).
//   {exchange} = the O / down partial sums are the only data crossing XCDs. Producers store
//         them as fp16 (half the bytes of fp32: the exchange is partly bandwidth-bound) with the
//         exchange parity in the lowest mantissa bit of every value; the
//         consumers (N1 / N2 / final norm) poll one 16-byte hint per source XCD (its last-written
//         values), then read everything and re-read any value whose parity is still stale, so no
//         grid-wide barrier exists anywhere.
//   (the reference runs 9 grid-wide barriers per layer: src/pi05/mk6.cu:301-497).
//   N1/N2/FINAL: rank r owns tokens r and r+32, each normed by the wave that owns its token tile
//        (waves 0 and 2 on ranks 0-15, waves 1 and 3 on ranks 16-31), so a tile's chain of
//        stages runs on one wave index across the XCD: sum the 8 XCD partials (layer 0 of a
//        step: the action embedding instead), gated residual (the residual x and x_t live in
//        LDS), adaRMS -> bf16 operand (or the final action projection and Euler update).
//   QKV: 768 rows per XCD (q rows of head g + all k and v rows), 24 rows per CU, RoPE epilogue.
//   ATT: head g, prefix keys split into 32 chunks (one per rank), the first 32 of a chunk from
//        the LDS ring pages the loader prefetched; this step's keys of tokens r and r+32 from the
//        XCD-private copies QKV writes, as one more block. MFMA S^T = K Q^T, online softmax,
//        O^T = V^T P^T; normalised partial O (bf16, whole operand fragments) with (m, l) per
//        chunk.
//   COMB: flash-decoding combine of the 32 chunk partials, one operand fragment of attn_g per
//        rank (four waves, eight chunks each, meeting in LDS); a wave waits only for the attention
//        waves of its eight chunks.
//   O:   W_o[32r..32r+32, 256g..256g+256) x attn_g -> partial o_g.
//   GU:  32 interleaved gate/up rows per CU -> gelu_tanh(g)*u -> h_g (bf16, XCD-private).
//   DN:  W_d[32r..32r+32, 512g..512g+512) x h_g -> partial z_g.
// GEMMs: v_mfma_f32_16x16x32_bf16, weight rows as the A operand (16 rows x 32 k per 1 KB
// fragment, read from the LDS ring in batches of eight ahead of their MFMAs) and the wave's 16
// tokens as B (16-byte sc1 loads from the XCD's L2, pipelined in chunks of 8 k-steps).
#include "fa_device.h"
#include "../../include/flashact_mi355x.h"
#include "fa_host.h"

#include <mutex>

namespace fa {
namespace pi05 {

constexpr int D = 1024, HD = 256, AD = 32;
constexpr int NX = 8, NR = 32, NWG = 256, TP = 64;
constexpr int NCW = 4, NLW = 2, NTH = 64 * (NCW + NLW);  // compute waves, loader waves
constexpr int NCH = 32;                                 // attention key chunks per head
constexpr int RING = 9, PAGE = 16384;                  // ring pages, page bytes
// Ring pages of one layer. With bf16 weights a weight page holds 16 fragments of 16 rows x 32 k
// (1 KB each); with fp8 weights it holds 16 fragment pairs of 16 rows x 64 k (the same 1 KB per
// copy instruction), so each weight kind needs half the pages. K and V^T pages are bf16 in both.
template <bool FP8>
struct Pages {
  static constexpr int QKV = 0, NQKV = FP8 ? 2 : 4;
  static constexpr int K = QKV + NQKV, V = K + 1, O = V + 1, GU = O + 1, NGU = FP8 ? 2 : 4;
  static constexpr int DN = GU + NGU, NDN = FP8 ? 1 : 2, PPL = DN + NDN;
};
constexpr int PPL_MAX = Pages<false>::PPL;
constexpr int MAXF = 1;                                 // pages in flight per loader wave
constexpr uint32_t OOB = 0x80000000u;                   // buffer offset past every resource

// workspace layout (bytes)
constexpr uint32_t OFF_CTRL = 0;     // u64 launch sequence, u32 error bits, u32 exchange parity base
constexpr uint32_t OFF_XFLAG = 1024; // [8 XCD][32 rank][4 wave] u64 epochs
// GEMM operands (xn, q, attention output, MLP activation h) are stored in MFMA fragment order:
// [XCD][token tile of 16][k-step of 32][token % 16][k % 32 / 8][8 bf16], so each 1 KB fragment a
// wave loads as the B operand is contiguous (see frag_off).
constexpr uint32_t OFF_XN = kWsDataBase;                                  // [8][4][32][16][4][8] bf16
constexpr uint32_t OFF_Q = OFF_XN + NX * TP * D * 2;                // [8][4][8][16][4][8] bf16
constexpr uint32_t OFF_ATTP = OFF_Q + NX * TP * HD * 2;             // [8][32 chunks][4][8][16][4][8] bf16
constexpr uint32_t OFF_ATTML = OFF_ATTP + NX * NCH * TP * HD * 2;   // [8][32][64][2] f32
constexpr uint32_t OFF_ATTN = OFF_ATTML + NX * NCH * TP * 2 * 4;    // [8][4][8][16][4][8] bf16
constexpr uint32_t OFF_H = OFF_ATTN + NX * TP * HD * 2;             // [8][4][16][16][4][8] bf16
constexpr uint32_t OFF_XP = OFF_H + NX * TP * 512 * 2;              // [2][8][64][1024] fp16, parity-tagged
// This step's own keys/values (the suffix), token t held by attention rank t % 32 as its slot t / 32:
// K [8 XCD][32 ranks][2 slots][256 dims] (one slot = one 512-byte key row, so a lane of the
// attention MFMA's A fragment loads 16 contiguous bytes) and V [8 XCD][32 ranks][16][16][2]
// (dim 16 dt + lr of both slots at ((rank 16 + lr) 16 + dt) 4 bytes: a lane's 16 dims are 64
// contiguous bytes).
constexpr uint32_t OFF_KS = OFF_XP + 2 * NX * TP * D * 2;
constexpr uint32_t OFF_VS = OFF_KS + NX * NR * 2 * HD * 2;
constexpr uint32_t WS_BYTES = OFF_VS + NX * NR * 2 * HD * 2;
static_assert(OFF_XFLAG + NX * NR * NCW * 8 <= kWsCounters, "flags stay below the fixup counters");

// LDS layout (bytes)
constexpr uint32_t L_CTL = RING * PAGE;        // u32 ready[2], consumed[4], abort, -, -, combine count
constexpr uint32_t L_XRES = L_CTL + 64;        // f32 [2][1024] residual stream of tokens r, r+32 (slot = wave / 2)
constexpr uint32_t L_XT = L_XRES + 2 * D * 4;  // f32 [2][32] x_t of tokens r, r+32
constexpr uint32_t L_COMB = L_XT + 2 * AD * 4;  // f32 [3][64][10] combine hand-off (waves 1-3 -> 0)
constexpr uint32_t LDS_BYTES = L_COMB + 3 * 64 * 10 * 4;
static_assert(LDS_BYTES <= 160 * 1024, "LDS of one CU");

// Byte offset of element (token t, k) of a fragment-ordered operand with KS k-steps of 32,
// relative to the XCD's block (XCD block size = 64 * 32 * KS * 2 bytes).
__host__ __device__ constexpr uint32_t frag_off(int KS, int t, int k) {
  return (uint32_t)(((((t >> 4) * KS + (k >> 5)) * 16 + (t & 15)) * 4 + ((k >> 3) & 3)) * 16 + (k & 7) * 2);
}

struct Params {
  const bf16* w1;  // bf16 weights, or e4m3 codes (fp8 launch) at the same addresses
  const bf16* wo;
  const bf16* w2;
  const bf16* w3;
  const float* s1;  // fp8 launch: per-row scales of the packed rows of w1, wo, w2, w3
  const float* so;
  const float* s2;
  const float* s3;
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
  unsigned long long* trace;
  unsigned char* ws;
  int NL, Lp, Lmax, S, Tv, xt_rows, trace_layer;
};

// Dynamic LDS of the kernel. Every LDS access goes through this array so the compiler keeps the
// LDS address space and emits ds_* instructions (a generic pointer would turn them into flat
// accesses that also wait on the vector-memory counter).
extern __shared__ __attribute__((aligned(16))) unsigned char fa_lds[];

struct Ctx {
  int g, r, wave, lane, lr, lq;
  int kb0;              // first key of this rank's attention chunk
  rsrc_t ws, kc, vc, rc, rs;
  uint32_t lds_addr;    // LDS address of fa_lds (for m0)
  unsigned* err;
  uint64_t e;           // epoch of this wave's latest XCD barrier
  unsigned long long* tr;  // this wave's 32 trace slots for the traced layer, else null
};

__device__ __forceinline__ void stamp(const Ctx& c, int i) {
  if (c.tr && c.lane == 0) c.tr[i] = __builtin_amdgcn_s_memrealtime();
}

// Lane indices pass through an empty asm at every stage boundary, so the compiler recomputes the
// addresses derived from them inside each stage instead of keeping them live across the whole
// layer (which pushes the kernel past 256 VGPRs into scratch spills on the hot path).
__device__ __forceinline__ void launder(Ctx& c) { asm volatile("" : "+v"(c.lane), "+v"(c.lr), "+v"(c.lq)); }

// LDS control words (ready[2], consumed[4], abort) shared by the loader and compute waves of a
// workgroup: relaxed workgroup-scope atomics, which compile to plain ds_read/ds_write (a volatile
// access would keep the generic address space and become a flat access).
__device__ __forceinline__ unsigned ctl_ld(int i) {
  return __hip_atomic_load(reinterpret_cast<unsigned*>(fa_lds + L_CTL) + i, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ void ctl_st(int i, unsigned v) {
  __hip_atomic_store(reinterpret_cast<unsigned*>(fa_lds + L_CTL) + i, v, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_WORKGROUP);
}

// ---------------------------------------------------------------- XCD barrier (per wave)
// A sync point: the wave drains its stores (they have reached L2) and publishes its epoch to its
// own flag slot. xcd_sync then waits for every compute wave of the XCD; a stage whose waves need
// only some producers waits for those instead (xcd_wait_ranks), so it starts as soon as its own
// inputs are complete rather than when the slowest wave of the XCD is done.
__device__ __forceinline__ void xcd_signal(const Params& p, Ctx& c) {
  __builtin_amdgcn_s_waitcnt(0);  // this wave's stores have reached L2
  c.e += 1;
  if (c.lane == 0)
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p.ws + OFF_XFLAG) + (c.g * NR + c.r) * NCW + c.wave, c.e,
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ void xcd_sync(const Params& p, Ctx& c) {
  xcd_signal(p, c);
  if (__hip_atomic_load(c.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & kErrSpin) return;
  const uint32_t off = OFF_XFLAG + c.g * (NR * NCW * 8) + c.lane * 16;
  for (unsigned it = 0;; ++it) {
    const u32x4 v = ldb128<kCpSc1>(c.ws, off);
    const uint64_t a = ((uint64_t)v[1] << 32) | v[0];
    const uint64_t b = ((uint64_t)v[3] << 32) | v[2];
    if (__builtin_amdgcn_ballot_w64(!(a >= c.e && b >= c.e)) == 0) break;
    if (it > kSpinCap) {
      if (c.lane == 0) atomicOr(c.err, kErrSpin);
      break;
    }
    __builtin_amdgcn_s_sleep(2);
  }
  asm volatile("" ::: "memory");  // loads after the barrier stay after it
}

// Waits until compute wave `wv` of ranks [r0, r0 + n) of this XCD (n <= 32) has passed the sync
// point this wave passed last (epoch c.e).
__device__ __forceinline__ void xcd_wait_ranks(const Ctx& c, int r0, int n, int wv) {
  if (__hip_atomic_load(c.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & kErrSpin) return;
  const bool mine = c.lane < n;
  const uint32_t off = mine ? OFF_XFLAG + ((c.g * NR + r0 + c.lane) * NCW + wv) * 8 : OOB;
  for (unsigned it = 0;; ++it) {
    const u32x2 v = ldb64<kCpSc1>(c.ws, off);
    const uint64_t a = ((uint64_t)v[1] << 32) | v[0];
    if (__builtin_amdgcn_ballot_w64(mine && a < c.e) == 0) break;
    if (it > kSpinCap) {
      if (c.lane == 0) atomicOr(c.err, kErrSpin);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  asm volatile("" ::: "memory");  // loads after the wait stay after it
}

// Waits for the norm waves that wrote the operand rows of this wave's token tile w (token t is
// normed by rank t % 32, wave t / 16: ranks 16 (w % 2) .. +15, wave w).
__device__ __forceinline__ void wait_norm_rows(const Ctx& c) { xcd_wait_ranks(c, 16 * (c.wave & 1), 16, c.wave); }

// ---------------------------------------------------------------- weight ring
// Compute wave side: wait until both loader waves have landed page pg; release pages < upto.
__device__ __forceinline__ void page_wait(const Ctx& c, int pg) {
  for (unsigned it = 0;; ++it) {
    const unsigned r0 = ctl_ld(0), r1 = ctl_ld(1);
    if ((int)min(r0, r1) > pg || ctl_ld(6)) break;
    if (it > kSpinCap) {
      ctl_st(6, 1u);
      if (c.lane == 0) atomicOr(c.err, kErrSpin);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  asm volatile("" ::: "memory");  // ring reads stay after the wait
}
__device__ __forceinline__ void page_release(const Ctx& c, int upto) {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's LDS reads have returned
  if (c.lane == 0) ctl_st(2 + c.wave, (unsigned)upto);
}

__device__ __forceinline__ void dma16(const void* g, uint32_t lds_addr) {
  // global_load_lds_dwordx4: lane i copies 16 bytes from g to LDS m0 + 16 i, so a fragment lands
  // in MFMA lane order. Inline asm keeps the compiler from draining these copies at waits it
  // inserts for other memory operations; m0 is saved and restored (the compiler reserves it).
  unsigned saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
               : "=&s"(saved)
               : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory");
}

__device__ __forceinline__ int qkv_row(int g, int vr) {
  return vr < 256 ? 256 * g + vr : (vr < 512 ? 2048 + (vr - 256) : 2304 + (vr - 512));
}

// Pages of one layer (i = page index within the layer). Loader wave lw copies fragments
// 8lw..8lw+7 of each page; fragment f lands at ring slot offset f*1024 in MFMA lane order.
//   0-3 QKV  (fragment F = 16i + f: row tile F/32, k-step F%32; 24 rows, tile 1 holds 8)
//   4   K    (F: key tile F/8, k-step F%8) of keys kb0..kb0+31 (rows past the prefix: key 0)
//   5   V^T  (F: dim tile; lane (lr, lq) holds keys kb0 + 8lq .. +8 of dim 16F + lr)
//   6   O    (F: row tile F/8, k-step F%8) of W_o[32r.., 256g..]
//   7-10 GU  (F = 16(i-7) + f: row tile F/32, k-step F%32)
//   11-12 DN (F = 16(i-11) + f: row tile F/16, k-step F%16)
// (fp8 weights: see loader_bases.) Within one wave's half page, fragment ff (0..7) of every kind
// sits at a fixed byte stride from fragment 0, and layer l at a fixed stride from layer 0, so each
// lane precomputes one base address per page kind. Lanes whose rows this CU does not use copy a row it does (QKV tile 1
// lanes 8-15, keys past the prefix), so every copy runs with a full exec mask.
struct LoaderBases {
  const unsigned char* b[PPL_MAX];
};

// fp8 pages: QKV / GU page i = row tile i, slot = pair of k-steps (loader wave lw copies pairs
// 8lw..8lw+7); O and DN: row tile lw, slot 8lw + pair (O has 4 pairs per row tile: slots
// 8lw+4..8lw+7 repeat 8lw..8lw+3 so every page is 16 copies). A lane copies 16 bytes of its row.
template <bool FP8>
__device__ __forceinline__ void loader_bases(const Params& p, const Ctx& c, int lw, LoaderBases& L) {
  using P = Pages<FP8>;
  const unsigned char* w1 = reinterpret_cast<const unsigned char*>(p.w1);
  const unsigned char* wo = reinterpret_cast<const unsigned char*>(p.wo);
  const unsigned char* w2 = reinterpret_cast<const unsigned char*>(p.w2);
  const unsigned char* w3 = reinterpret_cast<const unsigned char*>(p.w3);
  if constexpr (FP8) {
#pragma unroll
    for (int i = 0; i < P::NQKV; i++) {
      const int lr = (i == 1 && c.lr >= 8) ? c.lr - 8 : c.lr;
      L.b[P::QKV + i] = w1 + (size_t)qkv_row(c.g, 24 * c.r + i * 16 + lr) * D + 512 * lw + 16 * c.lq;
    }
    L.b[P::O] = wo + (size_t)(32 * c.r + 16 * lw + c.lr) * 2048 + 256 * c.g + 16 * c.lq;
#pragma unroll
    for (int i = 0; i < P::NGU; i++)
      L.b[P::GU + i] = w2 + (size_t)(1024 * c.g + 32 * c.r + 16 * i + c.lr) * D + 512 * lw + 16 * c.lq;
    L.b[P::DN] = w3 + (size_t)(32 * c.r + 16 * lw + c.lr) * 4096 + 512 * c.g + 16 * c.lq;
  } else {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int F0 = 16 * i + 8 * lw, rt = F0 >> 5, ks0 = F0 & 31;
      const int lr = (rt == 1 && c.lr >= 8) ? c.lr - 8 : c.lr;
      L.b[i] = w1 + ((size_t)qkv_row(c.g, 24 * c.r + rt * 16 + lr) * D + ks0 * 32 + c.lq * 8) * 2;
    }
    L.b[P::O] = wo + ((size_t)(32 * c.r + 16 * lw + c.lr) * 2048 + 256 * c.g + c.lq * 8) * 2;
#pragma unroll
    for (int i = P::GU; i < P::DN; i++) {
      const int F0 = 16 * (i - P::GU) + 8 * lw, rt = F0 >> 5, ks0 = F0 & 31;
      L.b[i] = w2 + ((size_t)(1024 * c.g + 32 * c.r + 16 * rt + c.lr) * D + ks0 * 32 + c.lq * 8) * 2;
    }
#pragma unroll
    for (int i = P::DN; i < P::PPL; i++)
      L.b[i] = w3 + ((size_t)(32 * c.r + 16 * (i - P::DN) + c.lr) * 4096 + 512 * c.g + 8 * lw * 32 + c.lq * 8) * 2;
  }
  {
    int key = c.kb0 + 16 * lw + c.lr;
    if (key >= p.Lp) key = 0;
    L.b[P::K] = reinterpret_cast<const unsigned char*>(p.kcache + (size_t)key * HD + c.lq * 8);
    // An 8-key group that starts inside the prefix is copied from its own row even when it runs
    // past Lp (it stays inside the row: Lmax >= 8 * ceil(Lp / 8)); keys >= Lp are masked by the
    // attention stage. Groups entirely past the prefix copy keys 0..7 instead.
    int kv = c.kb0 + 8 * c.lq;
    if (kv >= p.Lp) kv = 0;
    L.b[P::V] = reinterpret_cast<const unsigned char*>(p.vtcache + (size_t)(128 * lw + c.lr) * p.Lmax + kv);
  }
}

#define FA_VMCNT(n) (((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))
// Wait until at most 8n of this wave's copies are outstanding (copies complete in issue order).
__device__ __forceinline__ void vm_wait_pages(int n) {
  switch (n) {
    case 0: __builtin_amdgcn_s_waitcnt(FA_VMCNT(0)); break;
    case 1: __builtin_amdgcn_s_waitcnt(FA_VMCNT(8)); break;
    case 2: __builtin_amdgcn_s_waitcnt(FA_VMCNT(16)); break;
    case 3: __builtin_amdgcn_s_waitcnt(FA_VMCNT(24)); break;
    case 4: __builtin_amdgcn_s_waitcnt(FA_VMCNT(32)); break;
    case 5: __builtin_amdgcn_s_waitcnt(FA_VMCNT(40)); break;
    default: __builtin_amdgcn_s_waitcnt(FA_VMCNT(48)); break;
  }
  asm volatile("" ::: "memory");
}

// Loader wave main loop: pages are issued in launch order; page pg needs its ring slot free
// (every compute wave has released page pg - RING) and fewer than MAXF pages of this wave in
// flight. While it cannot issue, the wave completes its oldest page and publishes
// ready[lw] = number of pages landed. Ends when every page has landed (or on abort).
template <bool FP8>
__device__ void loader_main(const Params& p, const Ctx& c, int lw) {
  using P = Pages<FP8>;
  constexpr int PPL = P::PPL;
  constexpr size_t EB = FP8 ? 1 : 2;  // bytes per weight element
  LoaderBases L;
  loader_bases<FP8>(p, c, lw, L);
  const int NL = p.NL;
  const int total = p.S * NL * PPL;
  const size_t kvl = (size_t)p.Lmax * HD * 2;  // layer stride of both caches (bytes)
  const uint32_t vfs = 16u * p.Lmax * 2;       // V^T fragment stride: 16 dims
  int done = 0;
  bool ok = true;
  // diagnostics: issue / wait / landing time of each page of the traced layer (loader wave 0)
  unsigned long long* tr = (p.trace && lw == 0) ? p.trace + ((size_t)blockIdx.x * (NCW + 2) + NCW) * 32 : nullptr;
  const int tpg0 = p.trace_layer * PPL;
  auto complete_oldest = [&](int issued) {
    if (tr && c.lane == 0 && done >= tpg0 && done < tpg0 + PPL) tr[32 + done - tpg0] = __builtin_amdgcn_s_memrealtime();
    vm_wait_pages(issued - done - 1);
    if (tr && c.lane == 0 && done >= tpg0 && done < tpg0 + PPL)
      tr[2 * (done - tpg0) + 1] = __builtin_amdgcn_s_memrealtime();
    ++done;
    if (c.lane == 0) ctl_st(lw, (unsigned)done);
  };
#pragma unroll 1
  for (int li = 0; li < p.S * NL && ok; li++) {
    const int l = li - (li / NL) * NL;
#pragma unroll
    for (int i = 0; i < PPL; i++) {
      const int pg = li * PPL + i;
      // make room for page pg
      for (unsigned idle = 0;;) {
        if (pg - done < MAXF) {
          if (pg < RING) break;
          const unsigned m = min(min(ctl_ld(2), ctl_ld(3)), min(ctl_ld(4), ctl_ld(5)));
          if ((int)m >= pg - RING + 1) break;
        }
        if (done < pg) {
          complete_oldest(pg);
          idle = 0;
          continue;
        }
        if (ctl_ld(6) || ++idle > kSpinCap) {
          if (!ctl_ld(6)) {
            ctl_st(6, 1u);
            if (c.lane == 0) atomicOr(c.err, kErrSpin);
          }
          ok = false;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
      if (!ok) break;
      const size_t lstride = i < P::K ? (size_t)2560 * D * EB
                           : i <= P::V ? kvl
                           : i == P::O ? (size_t)D * 2048 * EB
                           : i < P::DN ? (size_t)8192 * D * EB
                                       : (size_t)D * 4096 * EB;
      const uint32_t fstride = i == P::V ? vfs : 64u;
      const int fmask = (FP8 && i == P::O) ? 3 : 7;  // fp8 O: 4 pairs per row tile, copied twice
      const unsigned char* src = L.b[i] + (size_t)l * lstride;
      const uint32_t dst = c.lds_addr + (uint32_t)(pg % RING) * PAGE + lw * 8 * 1024;
#pragma unroll
      for (int ff = 0; ff < 8; ff++) dma16(src + (ff & fmask) * fstride, dst + ff * 1024);
      if (tr && c.lane == 0 && pg >= tpg0 && pg < tpg0 + PPL) tr[2 * (pg - tpg0)] = __builtin_amdgcn_s_memrealtime();
    }
  }
  if (ok)
    while (done < total) complete_oldest(total);
  __builtin_amdgcn_s_waitcnt(0);
}

// ---------------------------------------------------------------- GEMM (one token tile)
// Eight e4m3 weights (k order in bytes 0..7) -> the eight bf16 of an MFMA operand. e4m3 values
// are exact in bf16, so the conversion (scale 1) is exact; the row scale is applied to the sums.
template <bool HI>
__device__ __forceinline__ unsigned cvt_fp8x2(unsigned w) {
  return __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, HI));
}
__device__ __forceinline__ u32x4 fp8x8_to_bf16(unsigned lo, unsigned hi) {
  return u32x4{cvt_fp8x2<false>(lo), cvt_fp8x2<true>(lo), cvt_fp8x2<false>(hi), cvt_fp8x2<true>(hi)};
}

// Attention operands: bf16, or fp16 when the caller's caches are fp16 (KV16), so the attention runs
// on the cached keys and values as the caller holds them (v_mfma_f32_16x16x32_f16), with q, this
// step's keys and values and the softmax weights in fp16 as well.
template <bool KV16>
__device__ __forceinline__ unsigned pack_kv(float a, float b) {
  if constexpr (KV16) return pack_f16x2(a, b);
  else return pack_bf16x2(a, b);
}
template <bool KV16>
__device__ __forceinline__ unsigned short kv_bits(float a) {
  if constexpr (KV16) return __builtin_bit_cast(unsigned short, (_Float16)a);
  else return bf16_bits(a);
}
template <bool KV16>
__device__ __forceinline__ f32x4 mfma_kv(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (KV16) return mfma16h(a, b, c);
  else return mfma16(a, b, c);
}

// acc[rt] = sum_k W[row tile rt][k] * X[token 16w+lr][k] over KS k-steps. bf16 weights: fragment
// F = rt*KS + ks is slot F%16 of ring page pg0 + F/16. fp8 weights: pair P = rt*PRT + ks/2 is slot
// P%16 of page pg0 + P/16; its 1 KB holds row lr, k 16q..16q+15 of the pair at byte 16 (lr + 16 q),
// so k-step ks reads 8 bytes at 16 lr + 256 (2 (ks%2) + lq/2) + 8 (lq%2). xoff = byte offset in the
// workspace of X[token][k = 8 lq] (OOB for tokens >= Tv: the loads return zeros); k-step ks adds
// XSTRIDE bytes.
struct NoWait {
  __device__ void operator()(int) const {}
};

template <int RT, int KS, int XSTRIDE = 64, bool FP8 = false, int PRT = KS / 2, class Wait = NoWait>
__device__ __forceinline__ void gemm_tok(f32x4 (&acc)[RT], const Ctx& c, int pg0, uint32_t xoff, int ts,
                                         const Wait& wait = Wait()) {
  // Software-pipelined in chunks of 8 k-steps: the loads of chunk i+1 are in flight while the
  // MFMAs of chunk i run, so compute starts as soon as the first operands arrive.
  constexpr int NPG = FP8 ? (RT * PRT + 15) / 16 : (RT * KS + 15) / 16;
  constexpr int KC = KS < 8 ? KS : 8;
  constexpr int NCK = KS / KC;
  u32x4 xf[2][KC];
  wait(0);  // the producers of chunk 0's operand rows are done
#pragma unroll
  for (int k = 0; k < KC; k++) xf[0][k] = ldb128<kCpSc1>(c.ws, xoff + k * XSTRIDE);
  // two accumulators per row tile (even / odd k-steps) keep four independent MFMA chains in flight
  f32x4 ac2[RT][2];
#pragma unroll
  for (int rt = 0; rt < RT; rt++) ac2[rt][0] = ac2[rt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  page_wait(c, pg0 + NPG - 1);
  stamp(c, ts);
  uint32_t slot[NPG];
  const uint32_t loff = FP8 ? 16 * c.lr + 256 * (c.lq >> 1) + 8 * (c.lq & 1) : c.lane * 16;
#pragma unroll
  for (int k = 0; k < NPG; k++) slot[k] = ((pg0 + k) % RING) * PAGE + loff;
#pragma unroll
  for (int ck = 0; ck < NCK; ck++) {
    if (ck + 1 < NCK) {
      wait(ck + 1);
#pragma unroll
      for (int k = 0; k < KC; k++) xf[(ck + 1) & 1][k] = ldb128<kCpSc1>(c.ws, xoff + ((ck + 1) * KC + k) * XSTRIDE);
    }
    __builtin_amdgcn_sched_barrier(0);
    // A fragments are read from LDS in batches of AB ahead of their MFMAs (left to itself the
    // compiler keeps about two reads in flight and every MFMA waits out an LDS round trip)
    constexpr int NA = KC * RT, AB = NA < 8 ? NA : 8;
#pragma unroll
    for (int h = 0; h < NA; h += AB) {
      u32x4 af[AB];
#pragma unroll
      for (int j = 0; j < AB; j++) {
        const int k = (h + j) / RT, rt = (h + j) % RT;
        if constexpr (FP8) {
          const int ks = ck * KC + k, P = rt * PRT + (ks >> 1);
          const u32x2 q = *reinterpret_cast<const u32x2*>(fa_lds + slot[P >> 4] + (P & 15) * 1024 + 512 * (ks & 1));
          af[j] = fp8x8_to_bf16(q[0], q[1]);
        } else {
          const int F = rt * KS + ck * KC + k;
          af[j] = *reinterpret_cast<const u32x4*>(fa_lds + slot[F >> 4] + (F & 15) * 1024);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < AB; j++) {
        const int k = (h + j) / RT, rt = (h + j) % RT;
        ac2[rt][k & 1] = mfma16(af[j], xf[ck & 1][k], ac2[rt][k & 1]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int rt = 0; rt < RT; rt++) acc[rt] = ac2[rt][0] + ac2[rt][1];
  stamp(c, ts + 1);
}

// ---------------------------------------------------------------- exchange (cross-XCD)
// Column d(k) + i (i < 4) of a norm-stage lane, k < 4: the lane's two 16-byte fp16 loads per source
// XCD cover columns 8 lane + 512 kk + 0..7 (kk < 2), four of them per k.
__device__ __forceinline__ int ncol(int lane, int k) { return 8 * lane + 512 * (k >> 1) + 4 * (k & 1); }

// Reads the 8 XCD partials of token t, columns 8*lane + 512kk + 0..7 (kk < 2), from exchange
// buffer buf (fp16, parity in the lowest mantissa bit).
// First polls one hint word per source XCD (the 16 bytes written last-in-order by rank 31) with
// a short sleep between polls, so waiting consumers put almost no load on the fabric; then loads
// everything once and re-reads (again with a sleep) only the 16-byte groups whose parity is
// still stale. Correctness rests on the per-value parity check, not on the hint.
__device__ __forceinline__ void xread(const Ctx& c, int buf, int t, unsigned par, u32x4 (&v)[NX][2], int ts) {
  const uint32_t b0 = OFF_XP + ((buf * NX * TP + t) * D + 8 * c.lane) * 2;
  {
    const uint32_t hint = c.lane < NX ? OFF_XP + (((buf * NX + c.lane) * TP + t) * D + D - 8) * 2 : OOB;
    for (unsigned it = 0;; ++it) {
      const u32x4 h = ldb128<kCpSc1>(c.ws, hint);
      if (__builtin_amdgcn_ballot_w64(c.lane < NX && mism16(h, par)) == 0) break;
      if ((it & 1023) == 1023 &&
          ((__hip_atomic_load(c.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & kErrSpin) || it > kSpinCap))
        break;
      __builtin_amdgcn_s_sleep(4);
    }
  }
#pragma unroll
  for (int gg = 0; gg < NX; gg++)
#pragma unroll
    for (int k = 0; k < 2; k++) v[gg][k] = ldb128<kCpSc1>(c.ws, b0 + (gg * TP * D + 512 * k) * 2);
  for (unsigned it = 0;; ++it) {
    if (c.tr && c.lane == 0) c.tr[ts == 26 ? 31 : 27] = it;  // traced layer: re-read rounds so far
    unsigned bad = 0;
#pragma unroll
    for (int gg = 0; gg < NX; gg++)
#pragma unroll
      for (int k = 0; k < 2; k++) bad |= (mism16(v[gg][k], par) != 0u ? 1u : 0u) << (gg * 2 + k);
    if (__builtin_amdgcn_ballot_w64(bad != 0) == 0) break;
    if ((it & 255) == 255) {
      if ((__hip_atomic_load(c.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & kErrSpin) || it > kSpinCap) {
        if (c.lane == 0) atomicOr(c.err, kErrSpin);
        break;
      }
    }
    __builtin_amdgcn_s_sleep(4);
#pragma unroll
    for (int gg = 0; gg < NX; gg++)
#pragma unroll
      for (int k = 0; k < 2; k++)
        if ((bad >> (gg * 2 + k)) & 1u) v[gg][k] = ldb128<kCpSc1>(c.ws, b0 + (gg * TP * D + 512 * k) * 2);
  }
  asm volatile("" ::: "memory");
  stamp(c, ts);
}

// ---------------------------------------------------------------- norm stages
// MODE 0: x = embed(x_t) (layer 0).  MODE 1: x += gate * sum_g part_g.  MODE 2: as 1, then the
// final norm, action projection and Euler update of x_t. Token t = r + 32 (wave / 2) (slot wave / 2
// of the rank's LDS residual rows), run by waves whose parity is r / 16; lane holds
// columns ncol(lane, k) + i (k, i < 4).
template <int MODE>
__device__ __forceinline__ void stage_norm(const Params& p, const Ctx& c, int buf, unsigned par, const float* gate,
                                           const float* scale, const float* shift, float dt) {
  const int t = c.r + 32 * (c.wave >> 1);
  float* xres = reinterpret_cast<float*>(fa_lds + L_XRES) + (c.wave >> 1) * D;
  float* xt = reinterpret_cast<float*>(fa_lds + L_XT) + (c.wave >> 1) * AD;
  f32x4 sc[4], sh[4], gt[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const int d = ncol(c.lane, k);
    sc[k] = *reinterpret_cast<const f32x4*>(scale + d);
    sh[k] = *reinterpret_cast<const f32x4*>(shift + d);
    if (MODE != 0) gt[k] = *reinterpret_cast<const f32x4*>(gate + d);
  }
  f32x4 x[4];
  if (MODE == 0) {
    // x = W_ain x_t + b_ain from coalesced 1 KB reads of W_ain [1024][32]: read j covers rows
    // 8j..8j+7 (lane L: row 8j + L/8, inputs 4 (L%8)..+3), an 8-lane DPP sum finishes each row,
    // whose value goes through this wave's residual rows in LDS to the lane layout below.
    const f32x4 xa = *reinterpret_cast<const f32x4*>(xt + 4 * (c.lane & 7));
    const float* W = p.w_ain + 4 * c.lane;
#pragma unroll 1
    for (int j0 = 0; j0 < D / 8; j0 += 8) {
      f32x4 w[8];
#pragma unroll
      for (int j = 0; j < 8; j++) w[j] = *reinterpret_cast<const f32x4*>(W + (size_t)(j0 + j) * 8 * AD);
#pragma unroll
      for (int j = 0; j < 8; j++) {
        float s = w[j][0] * xa[0] + w[j][1] * xa[1] + w[j][2] * xa[2] + w[j][3] * xa[3];
        s = dpp_f32<0xB1>(s) + s;   // lane ^ 1
        s = dpp_f32<0x4E>(s) + s;   // lane ^ 2
        s = dpp_f32<0x141>(s) + s;  // the other quad of the 8-lane group
        if ((c.lane & 7) == 0) xres[8 * (j0 + j) + (c.lane >> 3)] = s;
      }
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int d = ncol(c.lane, k);
      x[k] = *reinterpret_cast<const f32x4*>(xres + d) + *reinterpret_cast<const f32x4*>(p.b_ain + d);
    }
  } else {
    u32x4 v[NX][2];
    xread(c, buf, t, par, v, buf == 0 ? 26 : 25);
#pragma unroll
    for (int k = 0; k < 4; k++) {
      f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int gg = 0; gg < NX; gg++) {
        const unsigned lo = v[gg][k >> 1][2 * (k & 1)], hi = v[gg][k >> 1][2 * (k & 1) + 1];
        s += f32x4{h_lo(lo), h_hi(lo), h_lo(hi), h_hi(hi)};
      }
      const f32x4 xo = *reinterpret_cast<const f32x4*>(xres + ncol(c.lane, k));
      x[k] = xo + gt[k] * s;
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < 4; k++) ss += x[k][0] * x[k][0] + x[k][1] * x[k][1] + x[k][2] * x[k][2] + x[k][3] * x[k][3];
  const float rr = rsqrtf(wave_sum(ss) / (float)D + 1e-6f);
  f32x4 h[4];
#pragma unroll
  for (int k = 0; k < 4; k++) {
#pragma unroll
    for (int i = 0; i < 4; i++) h[k][i] = x[k][i] * rr * (1.0f + sc[k][i]) + sh[k][i];
  }
  if (MODE != 2) {
#pragma unroll
    for (int k = 0; k < 4; k++) {
      const int d = ncol(c.lane, k);
      *reinterpret_cast<f32x4*>(xres + d) = x[k];
      const u32x2 pk = {pack_bf16x2(h[k][0], h[k][1]), pack_bf16x2(h[k][2], h[k][3])};
      *reinterpret_cast<u32x2*>(p.ws + OFF_XN + c.g * (TP * D * 2) + frag_off(32, t, d)) = pk;
    }
  } else {
    // v[a] = h . W_aout[a] + b_aout[a]; x_t += dt * v   (8 outputs per batch of loads)
#pragma unroll 1
    for (int a0 = 0; a0 < AD; a0 += 8) {
      f32x4 wv[8][4];
#pragma unroll
      for (int a = 0; a < 8; a++)
#pragma unroll
        for (int k = 0; k < 4; k++)
          wv[a][k] = *reinterpret_cast<const f32x4*>(p.w_aout + (a0 + a) * D + ncol(c.lane, k));
#pragma unroll
      for (int a = 0; a < 8; a++) {
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < 4; k++)
          s += wv[a][k][0] * h[k][0] + wv[a][k][1] * h[k][1] + wv[a][k][2] * h[k][2] + wv[a][k][3] * h[k][3];
        s = wave_sum(s);
        if (c.lane == 0) xt[a0 + a] += dt * (s + p.b_aout[a0 + a]);
      }
    }
  }
}

// fp8 launch: the scales of four consecutive rows (one lane's output rows of a row tile).
__device__ __forceinline__ f32x4 row_scales(const float* s, size_t row0) { return *reinterpret_cast<const f32x4*>(s + row0); }

// ---------------------------------------------------------------- QKV
// q, this step's keys and values: bf16, or fp16 with KV16 (also the rows written into the caller's
// caches in the last step, which are then the caller's fp16 caches).
template <bool FP8, bool KV16>
__device__ __forceinline__ void stage_qkv(const Params& p, const Ctx& c, int l, int pg0, bool last) {
  const int t = 16 * c.wave + c.lr;
  const bool tv = t < p.Tv;
  const bool any = 16 * c.wave < p.Tv;
  // RoPE factors of my rows, issued ahead of the GEMM
  u32x2 cs[2], sn[2];
#pragma unroll
  for (int rt = 0; rt < 2; rt++) {
    const int vr0 = 24 * c.r + rt * 16 + 4 * c.lq;
    const uint32_t o = (tv && vr0 < 512) ? (t * 128 + ((vr0 & 255) >> 1)) * 4 : OOB;
    cs[rt] = ldb64<kCpPlain>(c.rc, o);
    sn[rt] = ldb64<kCpPlain>(c.rs, o);
  }
  f32x4 sc[2];
  if constexpr (FP8) {
#pragma unroll
    for (int rt = 0; rt < 2; rt++) {
      const int vr0 = (rt == 0 || c.lq < 2) ? 24 * c.r + rt * 16 + 4 * c.lq : 0;  // rows of this rank only
      sc[rt] = row_scales(p.s1, (size_t)l * 2560 + qkv_row(c.g, vr0));
    }
  }
  f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  if (any)
    gemm_tok<2, 32, 1024, FP8, 16>(acc, c, pg0, tv ? OFF_XN + c.g * (TP * D * 2) + frag_off(32, t, 8 * c.lq) : OOB,
                                   15, [&c](int ck) {
                                     if (ck == 0) wait_norm_rows(c);
                                   });
  page_release(c, pg0 + Pages<FP8>::NQKV);
  if constexpr (FP8) {
#pragma unroll
    for (int rt = 0; rt < 2; rt++) acc[rt] *= sc[rt];
  }
#pragma unroll
  for (int rt = 0; rt < 2; rt++) {
    if (rt == 1 && c.lq >= 2) continue;  // rows 24r+24.. belong to the next rank
    const f32x4 v = acc[rt];
    const int vr0 = 24 * c.r + rt * 16 + 4 * c.lq;
    if (vr0 >= 512) {
      if (!tv) continue;
      const int d = vr0 - 512;
      // value dims d..d+3 of this step's token t into the XCD's copy: rank t % 32, slot t / 32
      unsigned short* vf = reinterpret_cast<unsigned short*>(p.ws + OFF_VS) + ((c.g * NR + (t & 31)) * 16) * 32 + (t >> 5);
#pragma unroll
      for (int i = 0; i < 4; i++) vf[(((d + i) & 15) * 16 + ((d + i) >> 4)) * 2] = kv_bits<KV16>(v[i]);
      if (last && c.g == (l & 7)) {
        unsigned short* vr = reinterpret_cast<unsigned short*>(p.vtcache) + ((size_t)l * HD + d) * p.Lmax + p.Lp + t;
#pragma unroll
        for (int i = 0; i < 4; i++) vr[(size_t)i * p.Lmax] = kv_bits<KV16>(v[i]);
      }
      continue;
    }
    if (!tv) continue;
    const int j = (vr0 & 255) >> 1;  // RoPE pair index within the head
    const float c0 = as_f32(cs[rt][0]), c1 = as_f32(cs[rt][1]);
    const float s0 = as_f32(sn[rt][0]), s1 = as_f32(sn[rt][1]);
    const float lo0 = v[0] * c0 - v[1] * s0, hi0 = v[1] * c0 + v[0] * s0;
    const float lo1 = v[2] * c1 - v[3] * s1, hi1 = v[3] * c1 + v[2] * s1;
    const unsigned plo = pack_kv<KV16>(lo0, lo1), phi = pack_kv<KV16>(hi0, hi1);
    if (vr0 < 256) {
      const uint32_t qb = OFF_Q + c.g * (TP * HD * 2);
      *reinterpret_cast<unsigned*>(p.ws + qb + frag_off(8, t, j)) = plo;
      *reinterpret_cast<unsigned*>(p.ws + qb + frag_off(8, t, j + 128)) = phi;
    } else {
      // Every XCD keeps its own copy of this step's keys for attention (rank t % 32, slot t / 32).
      // The caller's cache rows (the reference leaves the last step's suffix K/V there) are written
      // in the last step only, by XCD l % 8.
      bf16* kf = reinterpret_cast<bf16*>(p.ws + OFF_KS) + ((c.g * NR + (t & 31)) * 2 + (t >> 5)) * HD;
      *reinterpret_cast<unsigned*>(kf + j) = plo;
      *reinterpret_cast<unsigned*>(kf + j + 128) = phi;
      if (last && c.g == (l & 7)) {
        bf16* kr = p.kcache + ((size_t)l * p.Lmax + p.Lp + t) * HD;
        *reinterpret_cast<unsigned*>(kr + j) = plo;
        *reinterpret_cast<unsigned*>(kr + j + 128) = phi;
      }
    }
  }
}

// ---------------------------------------------------------------- attention partials
// Head g, chunk r: the prefix keys [kbeg, kend) of the chunk (C = 32 ceil(Lp / 1024) keys per rank)
// in 32-key blocks -- the first from the LDS pages the loader prefetched, later ones from the
// caches -- then this step's keys of tokens r and r + 32 (those below Tv) from the XCD's suffix
// copies, as one more block. Spreading this step's keys over all ranks keeps every rank's stage the
// same length (measured: the two ranks that held all of them ran 4.6 us against 2.8 us); their
// loads are issued after the last prefix block's S^T MFMAs (issued with q instead, they keep 48
// more VGPRs live through the prefix blocks, and the stage measured slower). Keys past kend:
// S = -inf, V = 0.
template <bool KV16>
__device__ __forceinline__ void stage_att(const Params& p, const Ctx& c, int l, int pgk) {
  const int C = 32 * max(1, (p.Lp + 32 * NCH - 1) / (32 * NCH));
  const int kbeg = c.kb0, kend = min(kbeg + C, p.Lp);
  const int nsfx = (c.r < p.Tv ? 1 : 0) + (c.r + 32 < p.Tv ? 1 : 0);  // this step's keys of this rank
  const int t = 16 * c.wave + c.lr;
  const bool tv = t < p.Tv;
  if (16 * c.wave >= p.Tv) {
    page_release(c, pgk + 2);
    return;
  }
  const uint32_t pbase = ((c.g * NCH + c.r) * TP + t);
  if (kbeg >= kend && nsfx == 0) {  // empty chunk: weight 0 in the combine
    if (tv && c.lq == 0) {
      const f32x2 ml = {-1e30f, 0.f};
      *reinterpret_cast<f32x2*>(p.ws + OFF_ATTML + pbase * 8) = ml;
    }
    page_release(c, pgk + 2);
    return;
  }
  const float qscale = 1.4426950408889634f / 16.0f;  // log2(e) / sqrt(256)
  u32x4 qf[8];
  {
    const uint32_t qb = tv ? OFF_Q + c.g * (TP * HD * 2) + frag_off(8, t, 8 * c.lq) : OOB;
#pragma unroll
    for (int ks = 0; ks < 8; ks++) qf[ks] = ldb128<kCpSc1>(c.ws, qb + ks * 1024);
  }
  // this step's keys of this rank: K rows (slot = MFMA row lr < nsfx, other rows zero) and the two
  // slots of V for dims 16 dt + lr (lanes of quarter 0), requested by issue_suffix()
  u32x4 skf[8], svf[4];
  const uint32_t ks0 = OFF_KS + (c.g * NR + c.r) * (2 * HD * 2);
  const uint32_t vs0 = OFF_VS + ((c.g * NR + c.r) * 16 + c.lr) * 64;
  auto issue_suffix = [&]() {
#pragma unroll
    for (int ks = 0; ks < 8; ks++)
      skf[ks] = ldb128<kCpSc1>(c.ws, c.lr < nsfx ? ks0 + c.lr * (HD * 2) + (32 * ks + 8 * c.lq) * 2 : OOB);
#pragma unroll
    for (int j = 0; j < 4; j++) svf[j] = ldb128<kCpSc1>(c.ws, c.lq == 0 && nsfx > 0 ? vs0 + 16 * j : OOB);
  };
  page_wait(c, pgk + 1);
  stamp(c, 23);
  const uint32_t kslot = (pgk % RING) * PAGE, vslot = ((pgk + 1) % RING) * PAGE;

  float m = -1e30f, lsum = 0.f;
  f32x4 o[16];
#pragma unroll
  for (int dt = 0; dt < 16; dt++) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const uint32_t kl = (uint32_t)l * p.Lmax * HD * 2;  // layer base, kcache [Lmax][256]
  const uint32_t vl = (uint32_t)l * HD * p.Lmax * 2;  // layer base, vtcache [256][Lmax]
  const uint32_t vstep = 16 * p.Lmax * 2;             // 16 dims
  if (kbeg >= kend) issue_suffix();
  // One 32-key block; the first comes from the ring pages, later ones from the caches. The first is
  // peeled (`first` a compile-time constant): as an if / else inside the loop, the two arms became two
  // conditional blocks in sequence, and the compiler's waits in the page arm covered the loads of
  // the cache arm, i.e. waited out this step's suffix keys before the P V MFMAs they should overlap.
  auto block = [&](int kb, auto first_c) __attribute__((always_inline)) {
    constexpr bool first = decltype(first_c)::value;
    const int kg0 = kb + c.lq * 4;
    f32x4 s[2];
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
      u32x4 kf[8];
      const int key = kb + kt * 16 + c.lr;
      if constexpr (first) {  // the ring page
#pragma unroll
        for (int ks = 0; ks < 8; ks++)
          kf[ks] = *reinterpret_cast<const u32x4*>(fa_lds + kslot + (kt * 8 + ks) * 1024 + c.lane * 16);
      } else {
        const uint32_t rb = key < kend ? kl + key * HD * 2 + c.lq * 16 : OOB;
#pragma unroll
        for (int ks = 0; ks < 8; ks++) kf[ks] = ldb128<kCpPlain>(c.kc, rb + ks * 64);
      }
      __builtin_amdgcn_sched_barrier(0);  // the tile's fragments are all requested before its MFMAs
      f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 8; ks++) a = mfma_kv<KV16>(kf[ks], qf[ks], a);
      s[kt] = a;
    }
    if (kb + 32 >= kend) issue_suffix();  // last prefix block: this step's keys arrive under its P V
    if (c.tr) stamp(c, first ? 29 : 30);
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
    bmax = cols_max(bmax);
    const float mnew = fmaxf(m, bmax);
    const float alpha = exp2_w(m - mnew);
    m = mnew;
    float psum = 0.f;
    unsigned pk[4];
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
      float pv[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        pv[i] = exp2_w(s[kt][i] - m);
        psum += pv[i];
      }
      pk[kt * 2 + 0] = pack_kv<KV16>(pv[0], pv[1]);
      pk[kt * 2 + 1] = pack_kv<KV16>(pv[2], pv[3]);
    }
    psum = cols_sum(psum);
    lsum = lsum * alpha + psum;
    // B operand P^T: k-slot 8lq+i <-> key kg0+i (i<4), kg0+16+(i-4) (i>=4); V^T uses the same order
    const u32x4 pb = {pk[0], pk[1], pk[2], pk[3]};
    unsigned vm[2][2];  // zero V elements of keys >= kend inside a partially valid 4-key group
#pragma unroll
    for (int h2 = 0; h2 < 2; h2++) {
      const int nv = min(max(kend - (kg0 + 16 * h2), 0), 4);
      vm[h2][0] = nv >= 2 ? 0xffffffffu : (nv == 1 ? 0xffffu : 0u);
      vm[h2][1] = nv >= 4 ? 0xffffffffu : (nv == 3 ? 0xffffu : 0u);
    }
    // V^T operand (dim 16dt+lr, keys kg0 + 16h + (0..3)) in two halves of 8 dim tiles
#pragma unroll
    for (int half = 0; half < 2; half++) {
      __builtin_amdgcn_sched_barrier(0);
      u32x2 vf[8][2];
#pragma unroll
      for (int h2 = 0; h2 < 2; h2++) {
        const int kg = kg0 + 16 * h2;
        if constexpr (first) {  // the ring page
          const int o8 = 16 * h2 + 4 * c.lq;  // key offset within the 32-key block
          const uint32_t ad = vslot + (c.lr + 16 * (o8 >> 3)) * 16 + (o8 & 7) * 2 + half * 8 * 1024;
#pragma unroll
          for (int d8 = 0; d8 < 8; d8++) vf[d8][h2] = *reinterpret_cast<const u32x2*>(fa_lds + ad + d8 * 1024);
        } else {
          const uint32_t vo = kg < kend ? vl + c.lr * p.Lmax * 2 + kg * 2 + half * 8 * vstep : OOB;
#pragma unroll
          for (int d8 = 0; d8 < 8; d8++) vf[d8][h2] = ldb64<kCpPlain>(c.vc, vo + d8 * vstep);
        }
      }
      __builtin_amdgcn_sched_barrier(0);  // the half's V^T fragments are all requested before its MFMAs
#pragma unroll
      for (int d8 = 0; d8 < 8; d8++) {
        const int dt = half * 8 + d8;
        const u32x4 va = {vf[d8][0][0] & vm[0][0], vf[d8][0][1] & vm[0][1], vf[d8][1][0] & vm[1][0],
                          vf[d8][1][1] & vm[1][1]};
        o[dt] = mfma_kv<KV16>(va, pb, o[dt] * alpha);
      }
    }
  };
  if (kbeg < kend) {
    block(kbeg, std::true_type{});
#pragma unroll 1
    for (int kb = kbeg + 32; kb < kend; kb += 32) block(kb, std::false_type{});
  }
  if (nsfx > 0) {
    // This step's keys: one 16-key S^T tile whose rows 0 (token r) and 1 (token r + 32) are valid;
    // P^T k-slots 8lq + i hold keys 4lq + i (i < 4), so only slots 0, 1 of quarter 0 are non-zero,
    // and the V^T operand of lane (lr, quarter 0) is dim 16 dt + lr of both slots.
    f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 8; ks++) a = mfma_kv<KV16>(skf[ks], qf[ks], a);
    float sv[4], bmax = -1e30f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      sv[i] = (c.lq == 0 && i < nsfx) ? a[i] * qscale : -1e30f;
      bmax = fmaxf(bmax, sv[i]);
    }
    bmax = cols_max(bmax);
    const float mnew = fmaxf(m, bmax);
    const float alpha = exp2_w(m - mnew);
    m = mnew;
    float pv[4], psum = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      pv[i] = exp2_w(sv[i] - m);
      psum += pv[i];
    }
    psum = cols_sum(psum);
    lsum = lsum * alpha + psum;
    const u32x4 pb = {pack_kv<KV16>(pv[0], pv[1]), pack_kv<KV16>(pv[2], pv[3]), 0u, 0u};
    const unsigned slot_mask = nsfx == 2 ? 0xffffffffu : 0xffffu;  // slot 1 is stale without token r + 32
#pragma unroll
    for (int dt = 0; dt < 16; dt++) {
      const u32x4 va = {svf[dt >> 2][dt & 3] & slot_mask, 0u, 0u, 0u};
      o[dt] = mfma_kv<KV16>(va, pb, o[dt] * alpha);
    }
  }
  stamp(c, 24);
  page_release(c, pgk + 2);
  // O^T / l (bf16) in the O projection's operand order: fragment ks of this token tile holds dims
  // 32ks..32ks+31, slot (token, q) dims 32ks + 8q..+7. A lane holds dims 16dt + 4lq + i of token lr,
  // so slot q = lq/2 + 2 (lq%2) of tiles (2ks, 2ks+1) is completed by the lane ^ 16 partner's four
  // dims (one swap per dword), and every store writes one whole 1 KB fragment (its valid rows).
  {
    const float inv = lsum > 0.f ? 1.0f / lsum : 0.f;
    const bool odd = c.lq & 1;
    const uint32_t ob = OFF_ATTP + ((c.g * NCH + c.r) * (TP / 16) + c.wave) * 8192 +
                        (c.lr * 4 + (c.lq >> 1) + 2 * (c.lq & 1)) * 16;
#pragma unroll
    for (int ks = 0; ks < 8; ks++) {
      const unsigned a0 = pack_bf16x2(o[2 * ks][0] * inv, o[2 * ks][1] * inv);
      const unsigned a1 = pack_bf16x2(o[2 * ks][2] * inv, o[2 * ks][3] * inv);
      const unsigned b0 = pack_bf16x2(o[2 * ks + 1][0] * inv, o[2 * ks + 1][1] * inv);
      const unsigned b1 = pack_bf16x2(o[2 * ks + 1][2] * inv, o[2 * ks + 1][3] * inv);
      const LanePair s0 = swap16(a0, b0), s1 = swap16(a1, b1);
      if (tv)  // rows past Tv are never read (the combine gives them weight 0)
        *reinterpret_cast<u32x4*>(p.ws + ob + ks * 1024) = odd ? u32x4{s0.lo, s1.lo, b0, b1} : u32x4{a0, a1, s0.hi, s1.hi};
    }
  }
  if (tv && c.lq == 0) {
    const f32x2 ml = {m, lsum};
    *reinterpret_cast<f32x2*>(p.ws + OFF_ATTML + pbase * 8) = ml;
  }
}

// ---------------------------------------------------------------- combine
// attn_g[t] = sum_ch w_ch O_ch[t] with w_ch = l_ch 2^(m_ch - M) / sum l 2^(m - M). Rank r combines
// fragment r of the head's output (token tile r / 8, k-step r % 8): a lane owns one 16-byte slot
// (token 16 (r / 8) + lane / 4, 8 dims). Wave w takes chunks 8w..8w+7; waves 1-3 hand their partials
// (weighted sum, max, weight) to wave 0 through LDS, counted in control word 9.
__device__ __forceinline__ void stage_comb(const Params& p, const Ctx& c, int li) {
  const int tt = c.r >> 3, ks = c.r & 7;
  if (16 * tt >= p.Tv) return;
  const int t = 16 * tt + (c.lane >> 2);
  constexpr int NC = NCH / NCW;
  xcd_wait_ranks(c, NC * c.wave, NC, tt);  // the attention waves of this wave's chunks
  u32x4 v[NC];
  u32x2 ml[NC];
#pragma unroll
  for (int i = 0; i < NC; i++) {
    const int ch = NC * c.wave + i;
    // rows past Tv were never written: their loads are skipped (out of range returns zeros)
    v[i] = ldb128<kCpSc1>(c.ws, t < p.Tv ? OFF_ATTP + ((c.g * NCH + ch) * (TP / 16) + tt) * 8192 + ks * 1024 + c.lane * 16
                                         : OOB);
    ml[i] = ldb64<kCpSc1>(c.ws, t < p.Tv ? OFF_ATTML + ((c.g * NCH + ch) * TP + t) * 8 : OOB);
  }
  __builtin_amdgcn_sched_barrier(0);  // all loads in flight before the first use
  float mw = -1e30f;
#pragma unroll
  for (int i = 0; i < NC; i++) mw = fmaxf(mw, as_f32(ml[i][0]));
  float lw = 0.f, u[8];
#pragma unroll
  for (int e = 0; e < 8; e++) u[e] = 0.f;
#pragma unroll
  for (int i = 0; i < NC; i++) {
    // exp2f, not the bare exp2_w: with exp2_w this stage measured 0.85 us slower per layer
    const float w = as_f32(ml[i][1]) * exp2f(as_f32(ml[i][0]) - mw);
    lw += w;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const unsigned d = w != 0.f ? v[i][e] : 0u;  // empty chunks (and tokens past Tv) hold no partial
      u[2 * e] = fmaf(w, bf_lo(d), u[2 * e]);
      u[2 * e + 1] = fmaf(w, bf_hi(d), u[2 * e + 1]);
    }
  }
  float* xl = reinterpret_cast<float*>(fa_lds + L_COMB) + c.lane * 10;  // + 640 (w - 1)
  unsigned* cnt = reinterpret_cast<unsigned*>(fa_lds + L_CTL) + 9;
  if (c.wave > 0) {
    float* xw = xl + 640 * (c.wave - 1);
#pragma unroll
    for (int e = 0; e < 8; e++) xw[e] = u[e];
    xw[8] = mw;
    xw[9] = lw;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    if (c.lane == 0) __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    return;
  }
  for (unsigned it = 0;; ++it) {
    if (__hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= 3u * (unsigned)(li + 1) || ctl_ld(6)) break;
    if (it > kSpinCap) {
      ctl_st(6, 1u);
      if (c.lane == 0) atomicOr(c.err, kErrSpin);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  asm volatile("" ::: "memory");
  float M = mw;
#pragma unroll
  for (int w = 0; w < NCW - 1; w++) M = fmaxf(M, xl[640 * w + 8]);
  float f = exp2f(mw - M), L = lw * f;
#pragma unroll
  for (int e = 0; e < 8; e++) u[e] *= f;
#pragma unroll
  for (int w = 0; w < NCW - 1; w++) {
    const float* xw = xl + 640 * w;
    f = exp2f(xw[8] - M);
    L = fmaf(xw[9], f, L);
#pragma unroll
    for (int e = 0; e < 8; e++) u[e] = fmaf(xw[e], f, u[e]);
  }
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  u32x4 out;
#pragma unroll
  for (int e = 0; e < 4; e++) out[e] = pack_bf16x2(u[2 * e] * inv, u[2 * e + 1] * inv);
  *reinterpret_cast<u32x4*>(p.ws + OFF_ATTN + c.g * (TP * HD * 2) + (tt * 8 + ks) * 1024 + c.lane * 16) = out;
}

// ---------------------------------------------------------------- O projection (K-window g)
// Writes all 16 token slots of the tile (zeros past Tv) so every exchange slot carries the
// current parity.
template <bool FP8>
__device__ __forceinline__ void stage_oproj(const Params& p, const Ctx& c, int l, int pg, unsigned par) {
  const int t = 16 * c.wave + c.lr;
  const bool tv = t < p.Tv;
  f32x4 sc[2];
  if constexpr (FP8) {
#pragma unroll
    for (int rt = 0; rt < 2; rt++) sc[rt] = row_scales(p.so, (size_t)l * D + 32 * c.r + rt * 16 + 4 * c.lq);
  }
  f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  if (16 * c.wave < p.Tv)
    gemm_tok<2, 8, 1024, FP8, 8>(acc, c, pg, tv ? OFF_ATTN + c.g * (TP * HD * 2) + frag_off(8, t, 8 * c.lq) : OOB, 17,
                                 [&c](int) { xcd_wait_ranks(c, 8 * c.wave, 8, 0); });  // the combine of this tile
  page_release(c, pg + 1);
  if constexpr (FP8) {
#pragma unroll
    for (int rt = 0; rt < 2; rt++) acc[rt] *= sc[rt];
  }
  bool range = false;
#pragma unroll
  for (int rt = 0; rt < 2; rt++)
    stb64<kCpSc1>(c.ws, OFF_XP + (((0 * NX + c.g) * TP + t) * D + 32 * c.r + rt * 16 + 4 * c.lq) * 2,
                  tag16(tv ? acc[rt] : f32x4{0.f, 0.f, 0.f, 0.f}, par, range));
  if (__builtin_amdgcn_ballot_w64(range) != 0 && c.lane == 0) atomicOr(c.err, kErrRange);
}

// ---------------------------------------------------------------- gate/up (F-slice g)
template <bool FP8>
__device__ __forceinline__ void stage_gu(const Params& p, const Ctx& c, int l, int pg0) {
  const int t = 16 * c.wave + c.lr;
  const bool tv = t < p.Tv;
  if (16 * c.wave >= p.Tv) {
    page_release(c, pg0 + Pages<FP8>::NGU);
    return;
  }
  f32x4 sc[2];
  if constexpr (FP8) {
#pragma unroll
    for (int rt = 0; rt < 2; rt++)
      sc[rt] = row_scales(p.s2, (size_t)l * 8192 + 1024 * c.g + 32 * c.r + rt * 16 + 4 * c.lq);
  }
  f32x4 acc[2];
  gemm_tok<2, 32, 1024, FP8, 16>(acc, c, pg0, tv ? OFF_XN + c.g * (TP * D * 2) + frag_off(32, t, 8 * c.lq) : OOB,
                                 19, [&c](int ck) {
                                   if (ck == 0) wait_norm_rows(c);
                                 });
  page_release(c, pg0 + Pages<FP8>::NGU);
  if (!tv) return;
  if constexpr (FP8) {
#pragma unroll
    for (int rt = 0; rt < 2; rt++) acc[rt] *= sc[rt];
  }
  // h(f) = gelu(gate f) * up f for this CU's 16 columns f = 8rt + 2lq + (0, 1). One exchange with
  // lane ^ 16 gives every lane 4 consecutive columns, written as 8 bytes of the fragment-ordered h.
  const unsigned p0 = pack_bf16x2(gelu_tanh(acc[0][0]) * acc[0][1], gelu_tanh(acc[0][2]) * acc[0][3]);
  const unsigned p1 = pack_bf16x2(gelu_tanh(acc[1][0]) * acc[1][1], gelu_tanh(acc[1][2]) * acc[1][3]);
  const bool odd = c.lq & 1;
  const LanePair sw = swap16(p0, p1);  // even rows receive the odd partner's p0, odd rows the even partner's p1
  const unsigned recv = odd ? sw.lo : sw.hi;
  const u32x2 out = odd ? u32x2{recv, p1} : u32x2{p0, recv};
  const int f0 = odd ? 8 + 2 * (c.lq - 1) : 2 * c.lq;
  *reinterpret_cast<u32x2*>(p.ws + OFF_H + c.g * (TP * 512 * 2) + frag_off(16, t, 16 * c.r + f0)) = out;
}

// ---------------------------------------------------------------- down (K-window g)
template <bool FP8>
__device__ __forceinline__ void stage_dn(const Params& p, const Ctx& c, int l, int pg0, unsigned par) {
  const int t = 16 * c.wave + c.lr;
  const bool tv = t < p.Tv;
  f32x4 sc[2];
  if constexpr (FP8) {
#pragma unroll
    for (int rt = 0; rt < 2; rt++) sc[rt] = row_scales(p.s3, (size_t)l * D + 32 * c.r + rt * 16 + 4 * c.lq);
  }
  f32x4 acc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
  if (16 * c.wave < p.Tv)
    gemm_tok<2, 16, 1024, FP8, 8>(acc, c, pg0, tv ? OFF_H + c.g * (TP * 512 * 2) + frag_off(16, t, 8 * c.lq) : OOB,
                                  21, [&c](int ck) {
                                    // k-steps 8ck..8ck+7 are h columns 256ck.. of this XCD's F slice,
                                    // written by wave w of gate/up ranks 16ck..16ck+15
                                    xcd_wait_ranks(c, 16 * ck, 16, c.wave);
                                  });
  page_release(c, pg0 + Pages<FP8>::NDN);
  if constexpr (FP8) {
#pragma unroll
    for (int rt = 0; rt < 2; rt++) acc[rt] *= sc[rt];
  }
  bool range = false;
#pragma unroll
  for (int rt = 0; rt < 2; rt++)
    stb64<kCpSc1>(c.ws, OFF_XP + (((1 * NX + c.g) * TP + t) * D + 32 * c.r + rt * 16 + 4 * c.lq) * 2,
                  tag16(tv ? acc[rt] : f32x4{0.f, 0.f, 0.f, 0.f}, par, range));
  if (__builtin_amdgcn_ballot_w64(range) != 0 && c.lane == 0) atomicOr(c.err, kErrRange);
}

// ---------------------------------------------------------------- instrumentation
__device__ __forceinline__ void mark(const Params& p, const Ctx& c, int idx, uint64_t& t0) {
  if (p.stage_cycles && blockIdx.x == 0 && c.wave == 0 && c.lane == 0) {
    const uint64_t now = __builtin_amdgcn_s_memrealtime();
    p.stage_cycles[idx] += now - t0;  // 0-7 stages N1 QKV ATT COMB O N2 GU DN, 8 final, 9 XCD waits
    t0 = now;
  }
}

// ---------------------------------------------------------------- kernel
template <bool FP8, bool KV16>
__global__ void __launch_bounds__(NTH, 1) pi05_denoise_bs1(Params p) {
  using PG = Pages<FP8>;
  Ctx c;
  const int tid = threadIdx.x;
  c.lane = tid & 63;
  c.wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: derived offsets stay scalar
  c.lr = c.lane & 15;
  c.lq = c.lane >> 4;
  c.g = blockIdx.x & 7;
  c.r = blockIdx.x >> 3;
  c.kb0 = c.r * 32 * max(1, (p.Lp + 32 * NCH - 1) / (32 * NCH));
  c.ws = make_rsrc(p.ws, WS_BYTES);
  c.kc = make_rsrc(p.kcache, (uint32_t)((size_t)p.NL * p.Lmax * HD * 2));
  c.vc = make_rsrc(p.vtcache, (uint32_t)((size_t)p.NL * p.Lmax * HD * 2));
  c.rc = make_rsrc(p.rope_cos, (uint32_t)(p.Tv * 128 * 4));
  c.rs = make_rsrc(p.rope_sin, (uint32_t)(p.Tv * 128 * 4));
  c.lds_addr = (uint32_t)(uintptr_t)fa_lds;
  c.err = reinterpret_cast<unsigned*>(p.ws + OFF_CTRL + 8);
  if (tid < 16) ctl_st(tid, 0u);
  if (tid == 0 && xcc_id() != (unsigned)c.g) atomicOr(c.err, kErrXcd);
  const uint64_t seq = ld_flag(reinterpret_cast<const uint64_t*>(p.ws + OFF_CTRL));
  unsigned xbase =
      __hip_atomic_load(reinterpret_cast<const unsigned*>(p.ws + OFF_CTRL + 12), __ATOMIC_RELAXED,
                        __HIP_MEMORY_SCOPE_AGENT);
  const unsigned owner =
      __hip_atomic_load(reinterpret_cast<const unsigned*>(p.ws + kWsOwner), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();  // the only workgroup barrier: LDS control words are initialised
  if (c.wave >= NCW) {
    loader_main<FP8>(p, c, c.wave - NCW);
    return;
  }
  c.e = seq << 32;
  c.tr = nullptr;
  if (owner != kOwnerPi05Bs1) {
    // Another kernel used the workspace since this one last did: its data may sit in the exchange
    // buffers with any parity. The compute waves clear them (parity 0), restart the parity
    // sequence and pass one grid barrier before the first exchange.
    xbase = 0;
    constexpr uint32_t n16 = 2u * NX * TP * D * 2 / 16;
    for (uint32_t i = blockIdx.x * (NCW * 64) + tid; i < n16; i += NWG * NCW * 64)
      stb128<kCpSc1>(c.ws, OFF_XP + 16 * i, u32x4{0u, 0u, 0u, 0u});
    __builtin_amdgcn_s_waitcnt(0);
    c.e += 1;
    if (c.lane == 0)
      __hip_atomic_store(reinterpret_cast<uint64_t*>(p.ws + OFF_XFLAG) + (c.g * NR + c.r) * NCW + c.wave, c.e,
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    poll_flags(c.ws, OFF_XFLAG, NX * NR * NCW * 8, c.e, c.err);
  }
  const int NL = p.NL;
  const bool nw = (c.wave & 1) == (c.r >> 4) && c.r + 32 * (c.wave >> 1) < p.Tv;  // this wave owns a token in norm stages
  if (nw && c.lane < AD)
    reinterpret_cast<float*>(fa_lds + L_XT)[(c.wave >> 1) * AD + c.lane] = p.x_t[(c.r + 32 * (c.wave >> 1)) * AD + c.lane];

  const float dt = -1.0f / (float)p.S;
  uint64_t t0 = __builtin_amdgcn_s_memrealtime();
#pragma unroll 1
  for (int step = 0; step < p.S; step++) {
#pragma unroll 1
    for (int l = 0; l < NL; l++) {
      launder(c);
      const int li = step * NL + l;
      const int pb = li * PG::PPL;
      const unsigned par = (1u + xbase + (unsigned)li) & 1u;
      c.tr = (p.trace && li == p.trace_layer) ? p.trace + ((size_t)blockIdx.x * (NCW + 2) + c.wave) * 32 : nullptr;
      const float* mod_in = p.mods + ((size_t)li * 2 + 0) * 3 * D;
      const float* mod_post = p.mods + ((size_t)li * 2 + 1) * 3 * D;
      stamp(c, 0);
      const unsigned long long clk0 = c.tr ? __builtin_amdgcn_s_memtime() : 0ull;  // traced layer: shader clock
      if (nw) {
        if (l == 0)
          stage_norm<0>(p, c, 1, 0u, nullptr, mod_in, mod_in + D, 0.f);
        else
          stage_norm<1>(p, c, 1, par ^ 1u, mod_post - 6 * D + 2 * D, mod_in, mod_in + D, 0.f);
      }
      stamp(c, 1);
      mark(p, c, 0, t0);
      xcd_signal(p, c);  // QKV waves wait for the norm waves of their tile
      launder(c);
      mark(p, c, 9, t0);
      stamp(c, 2);
      stage_qkv<FP8, KV16>(p, c, l, pb + PG::QKV, step == p.S - 1);
      stamp(c, 3);
      mark(p, c, 1, t0);
      xcd_sync(p, c);
      launder(c);
      mark(p, c, 9, t0);
      stamp(c, 4);
      stage_att<KV16>(p, c, l, pb + PG::K);
      stamp(c, 5);
      mark(p, c, 2, t0);
      xcd_signal(p, c);  // combine waves wait for the attention waves of their chunks
      launder(c);
      mark(p, c, 9, t0);
      stamp(c, 6);
      stage_comb(p, c, li);
      stamp(c, 7);
      mark(p, c, 3, t0);
      xcd_signal(p, c);  // O waves wait for the combine of their tile
      launder(c);
      mark(p, c, 9, t0);
      stamp(c, 8);
      stage_oproj<FP8>(p, c, l, pb + PG::O, par);
      stamp(c, 9);
      mark(p, c, 4, t0);
      if (nw) stage_norm<1>(p, c, 0, par, mod_in + 2 * D, mod_post, mod_post + D, 0.f);
      stamp(c, 10);
      mark(p, c, 5, t0);
      xcd_signal(p, c);  // gate/up waves wait for the norm waves of their tile
      launder(c);
      mark(p, c, 9, t0);
      stamp(c, 11);
      stage_gu<FP8>(p, c, l, pb + PG::GU);
      stamp(c, 12);
      mark(p, c, 6, t0);
      xcd_signal(p, c);  // down waves wait, k-chunk by k-chunk, for the gate/up ranks of it
      launder(c);
      mark(p, c, 9, t0);
      stamp(c, 13);
      stage_dn<FP8>(p, c, l, pb + PG::DN, par);
      stamp(c, 14);
      if (c.tr && c.lane == 0) c.tr[28] = __builtin_amdgcn_s_memtime() - clk0;
      mark(p, c, 7, t0);
    }
    if (nw) {
      const int li = step * NL + NL - 1;
      const unsigned par = (1u + xbase + (unsigned)li) & 1u;
      const float* gl = p.mods + ((size_t)li * 2 + 1) * 3 * D + 2 * D;
      const float* mf = p.mod_final + (size_t)step * 3 * D;
      stage_norm<2>(p, c, 1, par, gl, mf, mf + D, dt);
    }
    mark(p, c, 8, t0);
  }
  if (c.g == 0 && nw && c.lane < AD)
    p.x_t[(c.r + 32 * (c.wave >> 1)) * AD + c.lane] = reinterpret_cast<float*>(fa_lds + L_XT)[(c.wave >> 1) * AD + c.lane];
  if (blockIdx.x == 0 && c.wave == 0 && c.lane == 0) {
    __hip_atomic_store(reinterpret_cast<unsigned*>(p.ws + OFF_CTRL + 12), (xbase + (unsigned)(p.S * NL)) & 1u,
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(reinterpret_cast<unsigned*>(p.ws + kWsOwner), kOwnerPi05Bs1, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p.ws + OFF_CTRL), seq + 1, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Scratch of fa_pi05_denoise_noalloc: one workspace in device memory reserved at load time, so
// that entry point never allocates. Host code reads its address per device with
// hipGetSymbolAddress and never uses this name as an address.
constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;
static_assert(WS_BYTES <= kNoAllocScratchBytes, "the batch-1 workspace fits the static scratch");
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

__global__ void ws_zero(u32x4* p, size_t n16) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x)
    p[i] = u32x4{0, 0, 0, 0};
}

}  // namespace pi05
}  // namespace fa
// ================================================================= host C ABI
using namespace fa;

extern "C" size_t fa_pi05_workspace_bytes(int batch, int Tv, int Lmax) {
  if (batch == 1) return pi05::WS_BYTES;
  if (batch < 1 || batch > fa_pi05_max_batch()) return 0;
  return pi05_batched_workspace_bytes(batch, Tv, Lmax);
}

extern "C" int fa_pi05_max_batch(void) { return 64; }

// Co-resident workgroups of the batch-1 bf16 kernel on `device`: occupancy per CU (at its thread
// count and dynamic LDS) times the CU count.
int fa::pi05_bs1_coop_capacity(int device) {
  int prev = 0;
  if (hipGetDevice(&prev) != hipSuccess) return 0;
  if (device != prev && hipSetDevice(device) != hipSuccess) return 0;
  int per_cu = 0, cus = 0;
  const void* kern = (const void*)pi05::pi05_denoise_bs1<false, false>;
  if (hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)pi05::LDS_BYTES) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, pi05::NTH, pi05::LDS_BYTES) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess)
    per_cu = 0;
  if (device != prev) (void)hipSetDevice(prev);
  return per_cu * cus;
}

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
  const bool fp8 = a->weight_dtype == FA_DTYPE_FP8_E4M3;
  if (!fp8 && a->weight_dtype != FA_DTYPE_BF16)
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: unknown weight_dtype=%d", a->weight_dtype);
  if (!fp8 && (a->s1 || a->so || a->s2 || a->s3))
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: fp8 row scales must be NULL for bf16 weights");
  if (fp8) {
    if (a->batch != 1)
      return host::fail(FA_ERR_UNSUPPORTED, "fa_pi05_denoise: fp8 weights are implemented for batch 1 (got batch=%d)",
                        a->batch);
    const float* sc[] = {a->s1, a->so, a->s2, a->s3};
    for (const float* x : sc) {
      if (!x) return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: fp8 weights need the row scales s1, so, s2, s3");
      if (reinterpret_cast<uintptr_t>(x) & 15)
        return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: fp8 row scales must be 16-byte aligned");
    }
  }
  if (a->srows < 0) return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: srows=%d < 0", a->srows);
  if (a->srows > 0) {  // K/V hand-off from a prefill's cache rows (src/pi05/mk6.cu:258-277)
    if (!a->kvsrc_k || !a->kvsrc_v)
      return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: srows > 0 needs kvsrc_k and kvsrc_v");
    if ((reinterpret_cast<uintptr_t>(a->kvsrc_k) | reinterpret_cast<uintptr_t>(a->kvsrc_v)) & 15)
      return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: kvsrc_k / kvsrc_v are not 16-byte aligned");
    if (a->srows < a->Lp)
      return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: srows=%d < Lp=%d hand-off rows", a->srows, a->Lp);
  }
  if (a->batch < 1 || a->batch > fa_pi05_max_batch())
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: batch=%d outside [1, %d]", a->batch, fa_pi05_max_batch());
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
  // The reference's fp16 caches at batch 1 without a hand-off: the batch-1 kernel reads and writes
  // them as they are and runs its attention in fp16 (no shadow).
  const bool kv16 = a->cache_dtype == FA_DTYPE_F16 && a->batch == 1 && a->srows == 0;
  if (a->cache_dtype == FA_DTYPE_F16 && !kv16) {
    // fp16 caches elsewhere (batch >= 2, or a hand-off): import into the bf16 shadow, run the bf16
    // loop on it, export the rows the loop wrote. Stream order sequences the three.
    const size_t need = fa_pi05_cache_shadow_bytes(a->batch, a->num_layers, a->Lmax);
    if (!a->cache_shadow || (reinterpret_cast<uintptr_t>(a->cache_shadow) & 255) || a->cache_shadow_bytes < need)
      return host::fail(FA_ERR_INVALID_ARG,
                        "fa_pi05_denoise: fp16 caches need a 256-byte aligned cache_shadow of >= %zu bytes "
                        "(got %p, %zu bytes)", need, a->cache_shadow, a->cache_shadow_bytes);
    fa_pi05_args b = *a;
    unsigned char* sh = static_cast<unsigned char*>(a->cache_shadow);
    b.kcache = sh;
    b.vtcache = sh + 2 * pi05_cache_elems(a->batch, a->num_layers, a->Lmax);
    b.cache_dtype = FA_DTYPE_BF16;
    b.cache_shadow = nullptr;
    b.cache_shadow_bytes = 0;
    int rc = pi05_cache_import(a, stream);
    if (rc == FA_OK) rc = fa_pi05_denoise(&b, stream);
    if (rc == FA_OK) rc = pi05_cache_export(a, stream);
    return rc;
  }
  if (a->cache_dtype != FA_DTYPE_BF16 && !kv16)
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: cache_dtype=%d is neither FA_DTYPE_BF16 nor FA_DTYPE_F16",
                      a->cache_dtype);
  if (a->batch > 1) return pi05_denoise_batched(a, stream);
  if (a->workspace_bytes < WS_BYTES)
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise: workspace_bytes=%zu < required %u", a->workspace_bytes,
                      (unsigned)WS_BYTES);
  const void* kern = fp8 ? (kv16 ? (const void*)pi05_denoise_bs1<true, true> : (const void*)pi05_denoise_bs1<true, false>)
                         : (kv16 ? (const void*)pi05_denoise_bs1<false, true> : (const void*)pi05_denoise_bs1<false, false>);
  int rc = host::check_device(kern, NTH, LDS_BYTES, NWG, "fa_pi05_denoise");
  if (rc != FA_OK) return rc;

  Params p;
  p.w1 = static_cast<const bf16*>(a->w1);
  p.wo = static_cast<const bf16*>(a->wo);
  p.w2 = static_cast<const bf16*>(a->w2);
  p.w3 = static_cast<const bf16*>(a->w3);
  p.s1 = a->s1;
  p.so = a->so;
  p.s2 = a->s2;
  p.s3 = a->s3;
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
  p.trace = a->trace;
  p.trace_layer = a->trace_layer;
  p.ws = static_cast<unsigned char*>(a->workspace);
  p.NL = a->num_layers;
  p.Lp = a->Lp;
  p.Lmax = a->Lmax;
  p.S = a->num_steps;
  p.Tv = a->Tv;
  p.xt_rows = a->xt_rows;
  if (a->srows > 0 && (rc = pi05_kv_handoff(a, stream)) != FA_OK) return rc;
  void* args[] = {&p};
  return host::coop_launch(kern, NWG, NTH, args, LDS_BYTES, stream, "fa_pi05_denoise");
}

// ---------------------------------------------------------------- no-allocation variant
namespace {
std::mutex g_scratch_mu;
void* g_scratch[64];  // device address of fa::pi05::scratch, per device ordinal (set on first use)
}  // namespace

extern "C" int fa_pi05_denoise_noalloc(const fa_pi05_args* a, fa_stream_t stream, void** scratch_out) {
  using namespace fa::pi05;
  if (!a) return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise_noalloc: args is NULL");
  if (a->workspace || a->workspace_bytes)
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise_noalloc: workspace must be NULL / 0 (this entry point "
                                          "uses the library's static scratch)");
  const size_t need = fa_pi05_workspace_bytes(a->batch, a->Tv, a->Lmax);
  if (need == 0 || need > kNoAllocScratchBytes)
    return host::fail(FA_ERR_INVALID_ARG, "fa_pi05_denoise_noalloc: batch=%d Tv=%d Lmax=%d needs a %zu-byte workspace; "
                      "the static scratch holds %zu bytes (use fa_pi05_denoise with a caller workspace)",
                      a->batch, a->Tv, a->Lmax, need, kNoAllocScratchBytes);
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return host::fail(FA_ERR_DEVICE, "fa_pi05_denoise_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= 64) return host::fail(FA_ERR_DEVICE, "fa_pi05_denoise_noalloc: device ordinal %d out of range", dev);
  void* ptr = nullptr;
  {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch[dev]) {
      // First call on this device (current): the scratch's device address, then a fill kernel
      // zeroes it on the caller's stream ahead of the first launch (the workspace's initial state).
      void* p = nullptr;
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(fa::pi05::scratch));
      if (e != hipSuccess || !p)
        return host::fail(FA_ERR_DEVICE, "fa_pi05_denoise_noalloc: hipGetSymbolAddress(scratch): %s",
                          hipGetErrorString(e));
      hipLaunchKernelGGL(ws_zero, dim3(1024), dim3(256), 0, (hipStream_t)stream, (u32x4*)p,
                         kNoAllocScratchBytes / 16);
      e = hipGetLastError();
      if (e != hipSuccess)
        return host::fail(FA_ERR_LAUNCH, "fa_pi05_denoise_noalloc: scratch init: %s", hipGetErrorString(e));
      g_scratch[dev] = p;
    }
    ptr = g_scratch[dev];
  }
  if (scratch_out) *scratch_out = ptr;
  fa_pi05_args b = *a;
  b.workspace = ptr;
  b.workspace_bytes = kNoAllocScratchBytes;
  return fa_pi05_denoise(&b, stream);
}
