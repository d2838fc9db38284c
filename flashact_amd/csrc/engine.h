// Stage engine of the batched denoise kernels and the prefix prefill (MFMA-bound regime: M = batch x
// Tv tokens, or the prefix tokens).
//
// One cooperative launch of 256 workgroups (one per CU) x NWAVE waves (4, or 8 where the kernel's
// source sets FA_ENG_NWAVE; see below). The loop is a
// fixed sequence of stages separated by grid barriers; inside a stage the workgroups take work
// items (GEMM tiles, attention blocks, rows) round robin in an XCD-major order, so consecutive
// items (which share a weight tile) run on the CUs of one XCD and hit that XCD's L2.
//
// Every intermediate crosses XCDs, so intermediates are stored with sc1 (write-through) and read
// with sc1 (buffer loads, or global_load_lds ... sc1 for GEMM operands); weights and the prefix
// K/V are read-only inputs.
#pragma once
#include <type_traits>

#include "fa_device.h"

namespace fa {
namespace eng {

// Waves per workgroup: 4 (one per SIMD, up to 512 VGPR + AGPR per lane) unless the kernel's source
// sets FA_ENG_NWAVE to 8 before including this header (two waves per SIMD, at most 256 registers per
// lane in every stage; a single wave keeps the MFMA pipe about 60 % busy, two about 85 %).
#ifndef FA_ENG_NWAVE
#define FA_ENG_NWAVE 4
#endif
constexpr int NWG = 256;                // workgroups (one per CU)
constexpr int NWAVE = FA_ENG_NWAVE;     // waves per workgroup
constexpr int NTHR = 64 * NWAVE;        // threads per workgroup
static_assert(NWAVE == 4 || NWAVE == 8, "4 or 8 waves per workgroup");

extern __shared__ __attribute__((aligned(16))) unsigned char lds[];

// With 8 waves (256 registers per lane) the thread index passes through an empty asm before anything
// is derived from it, so the compiler derives each stage's addresses inside the stage instead of
// hoisting them out of the layer loop and keeping them live across every other stage (8-wave
// prefill: 171 -> 20 spilled VGPRs; 0 with every thread-index use laundered, the uniform divisions
// below and the launch sequence number in SGPRs). With 4 waves the registers are there, and
// recomputing the addresses per stage measured slower (batch 16 19.09 -> 19.42 ms).
__device__ __forceinline__ int tid() {
  int t = threadIdx.x;
  if (NWAVE == 8) asm volatile("" : "+v"(t));
  return t;
}
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(tid() >> 6); }
__device__ __forceinline__ int lane_id() { return tid() & 63; }
// Thread 0 of workgroup 0. The thread test comes from tid() behind the workgroup test, so the two
// stay a scalar branch and a vector compare: folded into one compare, blockIdx.x gets a VGPR copy
// that its other uses then share.
__device__ __forceinline__ bool grid_thread0() { return blockIdx.x == 0 && tid() == 0; }
// 1 / d for a wave-uniform d (v_rcp_f32, 1 ulp), as an SGPR value: compute it where d is known,
// outside the loops that divide by it. The VGPR operand is laundered so that two calls do not share
// one reciprocal kept live (or spilled) between them.
__device__ __forceinline__ float rcp_u(int d) {
  asm volatile("" : "+v"(d));
  const float f = (float)d;
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, __builtin_amdgcn_rcpf(f))));
}
// m / d and m % d for 0 <= m < 2^20 and 0 < d, given rd = rcp_u(d): the float quotient, truncated,
// then one correction step (the compiler's integer expansion keeps its reciprocal in a VGPR).
struct QR {
  int q, r;
};
__device__ __forceinline__ QR divmod_u(int m, int d, float rd) {
  int q = (int)((float)m * rd), r = m - q * d;
  if (r < 0) {
    q -= 1;
    r += d;
  } else if (r >= d) {
    q += 1;
    r -= d;
  }
  return {q, r};
}
// XCD-major virtual workgroup index: workgroup b runs on XCD b % 8; v = xcd * 32 + rank.
__device__ __forceinline__ int vwg() {
  int v = (blockIdx.x & 7) * 32 + (blockIdx.x >> 3);
  if (NWAVE == 8) {
    asm volatile("" : "+v"(v));
    v = __builtin_amdgcn_readfirstlane(v);
  }
  return v;
}

// ---------------------------------------------------------------- global <-> LDS copies
// global_load_lds_dwordx4: lane i copies 16 bytes from its address to LDS m0 + 16 i, so one
// instruction lands one 1 KB MFMA fragment in lane order. m0 is saved and restored.
template <bool SC1>
__device__ __forceinline__ void dma16(const void* g, uint32_t lds_addr) {
  unsigned saved;
  if (SC1)
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, off sc1\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
                 : "memory");
  else
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(g), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
                 : "memory");
}

#define FA_ENG_VMCNT(n) (((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))
template <int N>
__device__ __forceinline__ void vm_wait() {
  __builtin_amdgcn_s_waitcnt(FA_ENG_VMCNT(N));
  asm volatile("" ::: "memory");
}

// The same copy with a wave-uniform 64-bit base in SGPRs and a 32-bit per-lane byte offset (one VGPR
// per copy address instead of two).
__device__ __forceinline__ void dma16s(const void* base, uint32_t voff, uint32_t lds_addr) {
  unsigned saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\tglobal_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
               : "=&s"(saved)
               : "v"(voff), "s"(base), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(uint32_t off) { return (uint32_t)(uintptr_t)lds + off; }
__device__ __forceinline__ u32x4 lds128(uint32_t off) { return *reinterpret_cast<const u32x4*>(lds + off); }

// sc1 stores through a buffer resource (base must be wave-uniform; offsets in bytes).
__device__ __forceinline__ void st_b128(rsrc_t r, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kCpSc1);
}
__device__ __forceinline__ void st_b64(rsrc_t r, uint32_t off, u32x2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, kCpSc1);
}
__device__ __forceinline__ void st_b32(rsrc_t r, uint32_t off, unsigned v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, r, off, 0, kCpSc1);
}
__device__ __forceinline__ void st_b16(rsrc_t r, uint32_t off, unsigned short v) {
  __builtin_amdgcn_raw_buffer_store_b16(v, r, off, 0, kCpSc1);
}
__device__ __forceinline__ rsrc_t rsrc_all(const void* base) { return make_rsrc(base, 0xffffffffu); }

// ---------------------------------------------------------------- grid barrier
// Two-level epoch barrier. Every workgroup stores its epoch to its slot of its XCD's 32 flags with
// a plain store (it stays in that XCD's L2); the XCD's rank-0 workgroup (the leader) polls those 32
// slots, publishes the XCD's epoch with a device-scope store to one of 8 slots, polls the 8, and
// releases its XCD through one more L2-local flag that the other 31 workgroups poll. Only the 8
// leaders touch cross-XCD flags, where a flat barrier had all 256 workgroups poll one 2 KB line:
// grid-barrier time per layer 25.1 -> 19.9 µs at pi0.5 batch 16 (23.2 -> 22.6 ms per launch);
// MolmoAct2 batch 16 45.8 -> 44.1 ms per launch.
// Flags: [8 XCD][32 rank] @0, XCD epochs [8] @2048, release flags [8] one line each @3072. The XCD
// of workgroup b must be b % 8 (checked by each kernel against HW_REG_XCC_ID; a mismatch sets
// kErrXcd, and the waits then run into their caps). Every wait is capped; a cap hit sets a sticky
// error bit that makes every later wait return at once.
struct Grid {
  uint64_t* flags;  // 4 KB of epoch flags (layout above)
  unsigned* err;
  uint64_t e;
};

struct NoSide {
  __device__ void operator()() const {}
};
// side(): run by waves 1.. while wave 0 waits at the barrier; work that needs nothing the barrier
// publishes (copies of launch inputs into LDS, which is free once the first workgroup barrier passed)
template <class F = NoSide>
__device__ __forceinline__ void grid_sync(Grid& g, const F& side = F{}) {
  __builtin_amdgcn_s_waitcnt(0);  // this wave's stores have completed
  __syncthreads();
  g.e += 1;
  const int t = tid();
  if (t >= 64) side();
  const int x = blockIdx.x & 7, rk = blockIdx.x >> 3, lane = t & 63;
  // flag stores through a wave-uniform descriptor (a generic pointer would keep the 64-bit address in
  // VGPRs across the whole layer loop)
  const rsrc_t r = make_rsrc(g.flags, 4096);
  const u32x2 ev = {(unsigned)g.e, (unsigned)(g.e >> 32)};
  if (t == 0)  // this XCD's slot (plain store: read back from the XCD's L2 by its leader)
    stb64<kCpPlain>(r, (uint32_t)(x * 32 + rk) * 8, ev);
  if (t < 64 && !(__hip_atomic_load(g.err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & kErrSpin)) {
    auto wait = [&](bool mine, uint32_t off) {
      for (unsigned it = 0;; ++it) {
        const u32x2 v = ldb64<kCpSc1>(r, mine ? off : 0x80000000u);
        if (__builtin_amdgcn_ballot_w64(mine && ((((uint64_t)v[1] << 32) | v[0]) < g.e)) == 0) break;
        if (it > kSpinCap) {
          if (lane == 0) atomicOr(g.err, kErrSpin);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
    };
    if (rk == 0) {  // XCD leader: its 32 workgroups, then the 8 XCD leaders, then release its XCD
      wait(lane < 32, (uint32_t)(x * 32 + lane) * 8);
      if (lane == 0) stb64<kCpSc1>(r, (uint32_t)(256 + x) * 8, ev);  // read by the other XCDs' leaders
      wait(lane < 8, (uint32_t)(256 + lane) * 8);
      if (lane == 0) stb64<kCpPlain>(r, (uint32_t)(384 + 16 * x) * 8, ev);
    } else {
      wait(lane == 0, (uint32_t)(384 + 16 * x) * 8);
    }
  }
  __syncthreads();
  asm volatile("" ::: "memory");
}

// ---------------------------------------------------------------- tiled GEMM
// A row-out epilogue's pack(n, v) or, when it takes its fetched inputs, pack(n, v, pre).
template <class E>
__device__ __forceinline__ auto pack_pre(const E& e, int n, f32x4 v, const typename E::Pre& p, int)
    -> decltype(e.pack(n, v, p)) {
  return e.pack(n, v, p);
}
template <class E>
__device__ __forceinline__ u32x4 pack_pre(const E& e, int n, f32x4 v, const typename E::Pre&, long) {
  return e.pack(n, v);
}
template <class E>
__device__ __forceinline__ u32x4 pack_pre(const E& e, int n, f32x4 v, const typename E::Pre& p) {
  return pack_pre(e, n, v, p, 0);
}

// C^T[n][m] = sum_k W[n][k] A[m][k] over k in [k0, k1) for a BM x BN tile (BM = 32 WM, BN = 32 WN).
// Waves form a 2 x 2 grid; wave (wm, wn) computes WM x WN MFMA blocks of 16 x 16 with
// v_mfma_f32_16x16x32_bf16 (A operand = 16 weight rows, B operand = 16 tokens), so after the loop
// lane l holds, for block (j, i), rows n = 16 (wn WN + j) + 4 (l / 16) + 0..3 of token
// m = 16 (wm WM + i) + l % 16 -- four consecutive output features of one token.
//
// Operands reach LDS by global_load_lds_dwordx4 in 128-wide k steps. A copy instruction that
// touches 8 or 16 rows streams at ~38 GB/s per CU; one that touches 4 rows x 256 B streams at
// ~145 GB/s (measured). So rows are taken in groups of 64: copy instruction r of a group loads
// rows r, r+16, r+32, r+48 (k step = 256 B each, 16 lanes per row) and lands them as 4 x 256 B at
// LDS pitch 1040 B. An MFMA fragment (16 rows of one 16-row block, 32 k) then reads row r from
// copy r at 1040 r + 256 (block % 4) + 64 ks + 16 q: the 16 rows fall in 16 different bank groups.
// Ring of RD steps (2, or 3 where three fit the kernel's LDS: two steps then stay in flight while one
// computes), one workgroup barrier per step. Rows m >= M copy row 0 (results discarded).
// With AF the activations are in MFMA fragment order instead (fragment (token block tb, k-step kk) =
// 1 KB at (tb lda / 32 + kk) * 1024, lane l = lr + 16 q holding token lr, k 8q..8q+7 at 16 l): copy f
// of a step is fragment (token block f / 4, k-step f % 4), one contiguous 1 KB, and lands whole in slot
// f, where the lane's operand is simply its own 16 bytes.
struct GemmArgs {
  const bf16* A;  // [M][lda] activations (written in this launch: sc1 copies)
  const bf16* W;  // [N][ldw] weights
  int lda, ldw, M;
};

template <int WM, int WN, bool AF = false>
struct GemmShape {
  static constexpr int BM = 32 * WM, BN = 32 * WN;
  static constexpr int GA = (BM + 63) / 64, GW = (BN + 63) / 64;  // 64-row groups
  // activation copies per step: 16 per 64-row group, or with AF one 1 KB fragment per 16 tokens and
  // 32 k (BM / 4: a 96-token tile copies 24, not the 32 of two 64-row groups)
  static constexpr int NA = AF ? BM / 4 : 16 * GA;
  static constexpr int NI = NA + 16 * GW;                         // copy instructions per step
  static constexpr int IPW = NI / NWAVE;                          // per wave
  static constexpr uint32_t PITCH = 1040;
  static constexpr uint32_t STEP = (uint32_t)NI * PITCH;
  static constexpr uint32_t LDS = 2 * STEP;
  static_assert(BN % 64 == 0, "weight tiles are whole 64-row groups");
  static_assert(NI % NWAVE == 0, "every wave issues the same number of copies");
};

template <int WM, int WN, bool AF = false, int RD = 2, class Epi>
__device__ __forceinline__ void gemm_tile(const GemmArgs& g, int m0, int n0, int k0, int k1, Epi& epi) {
  using S = GemmShape<WM, WN, AF>;
  const int w = wave_id(), lane = lane_id(), lr = lane & 15, lq = lane >> 4;
  const int wm = w & 1, wn = (w >> 1) & 1;
  // Waves 0-3 compute (2 x 2); with 8 waves, waves 4-7 share the copies and barriers only.
  const bool cw = NWAVE == 4 || w < 4;
  // this wave's copy instructions of every step: f = w + NWAVE j; lane -> (row slot lq, 16-byte chunk lr)
  const unsigned char* src[S::IPW];
#pragma unroll
  for (int j = 0; j < S::IPW; j++) {
    const int f = w + NWAVE * j;
    if (f < S::NA) {
      if constexpr (AF) {
        // blocks past the tile or past M copy the last token block of the operand (results discarded)
        int tb = (m0 >> 4) + (f >> 2);
        if (16 * (f >> 2) >= S::BM || 16 * tb >= g.M) tb = (g.M - 1) >> 4;
        src[j] = reinterpret_cast<const unsigned char*>(g.A) + ((size_t)tb * (g.lda >> 5) + (k0 >> 5) + (f & 3)) * 1024 +
                 16 * lane;
      } else {
        int row = m0 + 64 * (f >> 4) + 16 * lq + (f & 15);
        if (row >= g.M || 64 * (f >> 4) + 16 * lq >= S::BM) row = 0;
        src[j] = reinterpret_cast<const unsigned char*>(g.A + (size_t)row * g.lda + k0 + 8 * lr);
      }
    } else {
      const int fw = f - S::NA;
      const int row = n0 + 64 * (fw >> 4) + 16 * lq + (fw & 15);
      src[j] = reinterpret_cast<const unsigned char*>(g.W + (size_t)row * g.ldw + k0 + 8 * lr);
    }
  }
  const int ns = (k1 - k0) >> 7;
  auto issue = [&](int s) {
    const uint32_t base = (uint32_t)(s % RD) * S::STEP;
#pragma unroll
    for (int j = 0; j < S::IPW; j++) {
      const int f = w + NWAVE * j;
      if (f < S::NA)
        dma16<true>(src[j] + (AF ? 4096 : 256) * s, lds_addr(base + f * S::PITCH));
      else
        dma16<false>(src[j] + 256 * s, lds_addr(base + f * S::PITCH));
    }
  };
  f32x4 acc[WN][WM];
#pragma unroll
  for (int j = 0; j < WN; j++)
#pragma unroll
    for (int i = 0; i < WM; i++) acc[j][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  __builtin_amdgcn_s_waitcnt(0);  // earlier stores / loads of this wave are complete
  // Epilogue inputs (e.g. RoPE factors) are requested before the first copies, so their latency
  // passes under the prologue wait instead of after the last MFMA.
  typename Epi::Pre pre[WN][WM];
  if (cw) {
#pragma unroll
    for (int j = 0; j < WN; j++)
#pragma unroll
      for (int i = 0; i < WM; i++) {
        const int m = m0 + 16 * (wm * WM + i) + lr;
        pre[j][i] = epi.pre(n0 + 16 * (wn * WN + j) + 4 * lq, m < g.M ? m : 0);
      }
  }
  issue(0);
  if (RD > 2 && ns > 1) issue(1);
#pragma unroll 1
  for (int s = 0; s < ns; s++) {
    if (RD > 2 && s + 1 < ns)
      vm_wait<S::IPW>();  // step s + 1's copies (the last issued) may still be in flight
    else
      vm_wait<0>();
    __syncthreads();  // step s landed for every wave; every wave is done with step s - 1
    if (s + RD - 1 < ns) issue(s + RD - 1);
    if (!cw) continue;
    const uint32_t base = (uint32_t)(s % RD) * S::STEP;
    // fragments of k sub-step ks + 1 are read while the MFMAs of ks run (double-buffered)
    u32x4 a[2][WM], b[2][WN];
    auto rd = [&](int ks, int h) {
#pragma unroll
      for (int i = 0; i < WM; i++) {
        const int mb = wm * WM + i;  // 16-row block of A
        a[h][i] = AF ? lds128(base + (mb * 4 + ks) * S::PITCH + 16 * lane)
                     : lds128(base + (16 * (mb >> 2) + lr) * S::PITCH + (mb & 3) * 256 + ks * 64 + lq * 16);
      }
#pragma unroll
      for (int j = 0; j < WN; j++) {
        const int nb = wn * WN + j;
        b[h][j] = lds128(base + (S::NA + 16 * (nb >> 2) + lr) * S::PITCH + (nb & 3) * 256 + ks * 64 + lq * 16);
      }
    };
    rd(0, 0);
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
      if (ks + 1 < 4) rd(ks + 1, (ks + 1) & 1);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < WN; j++)
#pragma unroll
        for (int i = 0; i < WM; i++) acc[j][i] = mfma16(b[ks & 1][j], a[ks & 1][i], acc[j][i]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __syncthreads();  // the ring is free for the next tile
  if constexpr (Epi::kRowBytes > 0 && Epi::kStaged) {
    // Staged row-out epilogue: every lane packs its 4 features into OB bytes, the tile goes through
    // LDS (the ring is free), and each thread then stores 16 contiguous bytes of an output row, so
    // a store instruction writes whole lines (two 512-byte rows of fp32 partials, four 256-byte rows
    // of bf16 partials, or eight 128-byte rows of bf16 h) instead of 16 B into each of 16 rows.
    constexpr int OB = Epi::kRowBytes, RB = S::BN / 4 * OB, RP = RB + 16;
    static_assert(OB == 4 || OB == 8 || OB == 16, "4, 8 or 16 output bytes per 4 features");
    static_assert(S::BM * RP <= S::LDS, "the staged tile fits the ring");
    static_assert(RB % 16 == 0 && NTHR % (RB / 16) == 0, "whole rows per pass");
#pragma unroll
    for (int j = 0; j < WN; j++)
#pragma unroll
      for (int i = 0; i < WM && cw; i++) {
        const int ml = 16 * (wm * WM + i) + lr, nl = 16 * (wn * WN + j) + 4 * lq;
        const u32x4 v = pack_pre(epi, n0 + nl, acc[j][i], pre[j][i]);
        const uint32_t a = (uint32_t)(ml * RP + (nl >> 2) * OB);
        if constexpr (OB == 16)
          *reinterpret_cast<u32x4*>(lds + a) = v;
        else if constexpr (OB == 8)
          *reinterpret_cast<u32x2*>(lds + a) = u32x2{v[0], v[1]};
        else
          *reinterpret_cast<unsigned*>(lds + a) = v[0];
      }
    __syncthreads();
    constexpr int TPR = RB / 16, RPP = NTHR / TPR;  // threads per row, rows per pass
    const int t = tid(), tc = t % TPR;
#pragma unroll 4
    for (int r = t / TPR; r < S::BM; r += RPP) {
      const int m = m0 + r;
      if (m < g.M) st_b128(epi.ws, epi.row_off(m, n0) + (uint32_t)(tc * 16), lds128((uint32_t)(r * RP + tc * 16)));
    }
    __syncthreads();  // the staged tile is read before the next tile's copies land
  } else if constexpr (Epi::kRowBytes > 0) {
    // the same bytes stored in place: 16, 8 or 4 B into each of the 16 rows of an instruction
    constexpr int OB = Epi::kRowBytes;
#pragma unroll
    for (int j = 0; j < WN; j++)
#pragma unroll
      for (int i = 0; i < WM; i++) {
        const int ml = 16 * (wm * WM + i) + lr, nl = 16 * (wn * WN + j) + 4 * lq;
        if (cw && m0 + ml < g.M) {
          const u32x4 v = pack_pre(epi, n0 + nl, acc[j][i], pre[j][i]);
          const uint32_t o = epi.row_off(m0 + ml, n0) + (uint32_t)((nl >> 2) * OB);
          if constexpr (OB == 16)
            st_b128(epi.ws, o, v);
          else if constexpr (OB == 8)
            st_b64(epi.ws, o, u32x2{v[0], v[1]});
          else
            st_b32(epi.ws, o, v[0]);
        }
      }
  } else {
#pragma unroll
    for (int j = 0; j < WN; j++)
#pragma unroll
      for (int i = 0; i < WM; i++) {
        const int m = m0 + 16 * (wm * WM + i) + lr;
        if (cw && m < g.M) epi(n0 + 16 * (wn * WN + j) + 4 * lq, m, acc[j][i], pre[j][i]);
      }
  }
}

// Epilogue base for epilogues without per-element inputs. An epilogue that sets kRowBytes (4, 8
// or 16: output bytes per 4 consecutive features) instead provides pack(n, v) (the bytes of features
// n..n+3, in the low words) and row_off(m, n0) (byte offset in `ws` of row m's features from the
// tile's first feature n0); with kStaged, gemm_tile writes its rows whole through LDS (measured:
// MolmoAct2 batch 16 46.3 -> 45.1 ms, prefill 6.71 -> 6.64 ms; the batch-16 pi0.5 kernel, whose
// tiles are half as deep in k, ran 2 % slower staged and stores in place).
struct NoPre {
  struct Pre {};
  static constexpr int kRowBytes = 0;
  static constexpr bool kStaged = false;
  __device__ Pre pre(int, int) const { return Pre{}; }
};

// Runs every tile of an [M x N] GEMM, K split into `ksplit` equal ranges (multiples of 128). Items
// are ordered m-tile fastest so the items of one weight tile run on neighbouring CUs of one XCD.
// The epilogue receives the split index through epi.split.
// This workgroup's first item of a stage whose items come in groups of gs consecutive items sharing a
// weight tile. With at least NWG items: the XCD-major order vwg(). With fewer, XCD x takes the
// contiguous run of groups [ng x / 8, ng (x + 1) / 8), so every XCD runs about items / 8 of them where
// the XCD-major order fills XCDs 0, 1, .. and leaves the last ones idle; a group's items stay on one
// XCD, whose L2 serves the weight tile's later reads, and neighbouring groups (the same k range)
// share their activation tiles there too. Returns items for an idle workgroup; falls back to vwg()
// when an XCD's run of groups would not fit its 32 workgroups.
__device__ __forceinline__ int first_item(int items, int gs) {
  const int ng = (items + gs - 1) / gs;
  if (items >= NWG || (ng + 7) / 8 * gs > 32) return vwg();
  const int x = blockIdx.x & 7, r = blockIdx.x >> 3;
  const int it = ng * x / 8 * gs + r;
  return it < min(ng * (x + 1) / 8 * gs, items) ? it : items;
}

// XB: items placed by first_item (batched MolmoAct2: 34.13 -> 33.34 ms per launch at batch 16; the
// pi0.5 batched kernel's O and down projections, 224 items each: 19.17 -> 18.98 ms). The pi0.5 QKV
// stage (15.1 -> 15.5 us per layer with it) and the prefill (no change) keep vwg().
template <int WM, int WN, bool AF = false, int RD = 2, bool XB = false, class Epi>
__device__ __forceinline__ void gemm_stage(const GemmArgs& g, int N, int K, int ksplit, Epi& epi) {
  using S = GemmShape<WM, WN, AF>;
  const int nm = (g.M + S::BM - 1) / S::BM, nn = N / S::BN;
  const int items = nm * nn * ksplit, kc = K / ksplit;
#pragma unroll 1
  for (int it = XB ? first_item(items, nm) : vwg(); it < items; it += NWG) {
    const int mt = it % nm, rest = it / nm, nt = rest % nn, sp = rest / nn;
    epi.split = sp;
    gemm_tile<WM, WN, AF, RD>(g, mt * S::BM, nt * S::BN, sp * kc, sp * kc + kc, epi);
  }
}

// ---------------------------------------------------------------- direct-operand GEMM tiles
// gemm_tile_d<TW, WM>: a (16 WM TW)-token x 128-feature tile whose token operand skips LDS. The NWAVE
// waves form TW rows along the tokens and NWAVE / TW columns along the features; wave (wt, wf) computes
// WM token blocks x WN feature blocks of 16 x 16. The tall tile (TW = NWAVE, WM = 4: 256 x 128 with 4
// waves, 512 x 128 with 8; a wave holds 64 tokens x 128 features, 32 MFMAs per 32-k sub-step for 12
// fragment reads, against 16 for 8 in gemm_tile) is for GEMMs with many output tiles; the square one
// (4 waves, TW = 2: 128 or 96 x 128, the shape of gemm_tile) for the rest.
// * Activations are stored in MFMA fragment order (fragment (token block tb, k-step kk) = 1 KB at
//   (tb KF + kk) * 1024, lane l = lr + 16 q holding token lr, k 8q..8q+7 at 16 l) and loaded straight
//   into registers, a whole 128-k step ahead of their use (the waves of one token row load the same
//   fragments; each is used by one wave of the tall tile).
// * The weights go through a 4-stage LDS ring (the 4-row x 256 B copies of gemm_tile) filled three
//   steps ahead.
// * The loads of later steps are issued between the MFMAs instead of in one burst before them, which
//   at one wave per SIMD would stall the MFMA issue behind the copy queue: the weight copies during
//   sub-steps 0-1, and after each sub-step the next step's WM activation fragments of that sub-step,
//   into the registers its MFMAs have just read (one activation register set: 16 WM VGPRs, which keeps
//   the persistent kernels free of spills; two sets spilled 32-60 VGPRs in the prefill).
// Measured in isolation on L2-resident operands (a standalone probe, 256 CUs): the tall tile 7.5 µs
// per 128 x 128 x 1024 of work against 10.2-10.6 µs for gemm_tile; in the prefill kernel, gate/up
// 181 -> 114 µs and down 86 -> 62 µs per layer (128 x 128 tiles -> this tile).
struct GemmArgsF {
  rsrc_t A;        // fragment-ordered activations, bounded to ceil(M / 16) token blocks (loads past: 0)
  const bf16* W;   // [N][ldw] weights
  int KF, ldw, M;  // KF = the activation's K / 32 (fragments per token block)
};
constexpr uint32_t TALL_ST = 32 * 1040;   // one weight stage: 32 copies of 4 rows x 256 B
constexpr uint32_t TALL_LDS = 4 * TALL_ST;

template <class E, class = void>
struct HasPre : std::false_type {};
template <class E>
struct HasPre<E, std::void_t<typename E::Pre>> : std::true_type {};
template <class E, class = void>
struct IsStaged : std::false_type {};
template <class E>
struct IsStaged<E, std::void_t<decltype(E::kStaged)>> : std::bool_constant<E::kStaged && (E::kRowBytes > 0)> {};

// LDS bytes of gemm_tile_d<TW, WM>'s staged epilogue (8 output bytes per 4 features, 16 B row padding)
template <int TW, int WM>
constexpr uint32_t staged_d_lds() {
  return (uint32_t)NWAVE * 16 * WM * (128 / (NWAVE / TW) / 4 * 8 + 16);
}

// Epilogue: epi(n, m, v) with features n..n+3 of token m (m < M only); an epilogue with a Pre type
// (gemm_tile's interface) gets epi(n, m, v, pre) with every block's pre fetched before the first call.
template <int TW, int WM, class Epi>
__device__ __forceinline__ void gemm_tile_d(const GemmArgsF& g, int m0, int n0, int k0, int k1, Epi& epi) {
  static_assert(NWAVE % TW == 0 && (NWAVE / TW == 1 || NWAVE / TW == 2), "TW waves along the tokens");
  // FW waves along the features; CPW weight copies per wave and step, CPK of them in each of the
  // step's first two sub-steps (one every JM feature blocks)
  constexpr int FW = NWAVE / TW, WN = 8 / FW, NA = 4 * WM, CPW = 32 / NWAVE, CPK = CPW / 2, JM = WN / CPK;
  static_assert(JM >= 1 && WN % CPK == 0, "copy schedule");
  const int w = wave_id(), lane = lane_id(), lr = lane & 15, lq = lane >> 4;
  const int wt = w / FW, wf = w % FW;
  // copy f = w + NWAVE j of a step: rows 64 (f / 16) + 16 lq + f % 16 of the tile, 16 B per lane
  // (readfirstlane returns int: each half is cast to uint32_t before widening, or a low word with
  // bit 31 set would sign-extend over the high word)
  const uint64_t wb = reinterpret_cast<uint64_t>(g.W + (size_t)n0 * g.ldw);
  const uint32_t wlo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)wb);
  const uint32_t whi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(wb >> 32));
  const void* wbase = reinterpret_cast<const void*>(((uint64_t)whi << 32) | wlo);
  const uint32_t wlane = (uint32_t)((16 * lq * g.ldw + k0 + 8 * lr) * 2);
  const int tb0 = (m0 >> 4) + WM * wt;  // the wave's first token block
  const uint32_t abase = (uint32_t)(((size_t)tb0 * g.KF + (k0 >> 5)) * 1024 + lane * 16);
  const int ns = (k1 - k0) >> 7;
  f32x4 acc[WN][WM];
#pragma unroll
  for (int j = 0; j < WN; j++)
#pragma unroll
    for (int i = 0; i < WM; i++) acc[j][i] = f32x4{0.f, 0.f, 0.f, 0.f};
  u32x4 a[NA];  // [WM ks + i]: token block tb0 + i, k-step ks of the current 128-k step
  auto issue_w = [&](int s, int j) {
    const int f = w + NWAVE * j;
    dma16s(wbase, wlane + (uint32_t)((64 * (f >> 4) + (f & 15)) * g.ldw * 2 + 256 * s),
           lds_addr((uint32_t)(s & 3) * TALL_ST + f * 1040));
  };
  // Token blocks past M read zeros (the descriptor's bound) and their MFMAs run on them: no branch
  // in the loop, whose basic blocks the compiler would otherwise split at every load and MFMA group.
  auto load_a = [&](int s, int q) {
    a[q] = ldb128<kCpSc1>(g.A, abase + (uint32_t)(((q % WM) * g.KF + 4 * s + q / WM) * 1024));
  };
  __builtin_amdgcn_s_waitcnt(0);  // earlier stores / loads of this wave are complete
#pragma unroll
  for (int s = 0; s < 3; s++)
    if (s < ns)
#pragma unroll
      for (int j = 0; j < CPW; j++) issue_w(s, j);
#pragma unroll
  for (int q = 0; q < NA; q++) load_a(0, q);
  vm_wait<0>();
  __syncthreads();
  // One 128-k step on ring stage s % 4. The weight copies of step s + 3 go out during sub-steps 0-1;
  // once sub-step ks's MFMAs have read their WM activation fragments, the same registers take the
  // next step's fragments of sub-step ks (a whole step ahead of their use).
#pragma unroll 1
  for (int s = 0; s < ns; s++) {
    const uint32_t base = (uint32_t)(s & 3) * TALL_ST;
    // one fragment register set: fragment j of sub-step ks + 1 is read right after the MFMAs that
    // used fragment j of sub-step ks
    u32x4 wfr[WN];
    auto rd = [&](int ks, int j) {
      const int nb = wf * WN + j;  // 16-row feature block of the tile
      return lds128(base + (16 * (nb >> 2) + lr) * 1040 + (nb & 3) * 256 + ks * 64 + lq * 16);
    };
#pragma unroll
    for (int j = 0; j < WN; j++) wfr[j] = rd(0, j);
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
#pragma unroll
      for (int j = 0; j < WN; j++) {
        if (ks < 2 && j % JM == 0 && s + 3 < ns) issue_w(s + 3, CPK * ks + j / JM);
#pragma unroll
        for (int i = 0; i < WM; i++) acc[j][i] = mfma16(wfr[j], a[WM * ks + i], acc[j][i]);
        if (ks + 1 < 4) wfr[j] = rd(ks + 1, j);
      }
      // Unconditional (the last step's loads read past k1: another split's fragments, or zeros
      // past the descriptor's bound, never used). Behind a branch, the compiler's wait analysis
      // (which does not pair the branches of one condition) waited for every outstanding load,
      // the weight copy just issued included, before the first MFMAs of each step.
#pragma unroll
      for (int i = 0; i < WM; i++) load_a(s + 1, WM * ks + i);
      __builtin_amdgcn_sched_barrier(0);
    }
    // Everything but this step's loads has landed: stage (s + 1) % 4 (copied two steps ago) for this
    // wave; the barrier makes it every wave's and frees stage s % 4.
    if (s + 3 < ns)
      vm_wait<CPW + NA>();
    else
      vm_wait<NA>();
    __syncthreads();
  }
  if constexpr (!HasPre<Epi>::value && IsStaged<Epi>::value) {
    // Staged row-out epilogue, per wave: the wave's 16 WM token rows x (128 / FW) features go through
    // its own LDS rows (the ring is free once every wave's last MFMAs are done), then each lane
    // stores 16 contiguous bytes of a row, so an instruction writes whole row segments (four 256-byte
    // rows of bf16 partials) instead of 8 B into each of 16 rows. The kernel's LDS must hold
    // staged_d_lds<TW, WM>() bytes.
    constexpr int OB = Epi::kRowBytes, RB = 128 / FW / 4 * OB, RP = RB + 16, WR = 16 * WM;
    static_assert(OB == 8 && RB % 16 == 0 && 64 % (RB / 16) == 0, "8 output bytes per 4 features");
    __syncthreads();  // every wave's last MFMAs have read the ring
    if (16 * tb0 < g.M) {
      const uint32_t base = (uint32_t)w * WR * RP;
#pragma unroll
      for (int j = 0; j < WN; j++)
#pragma unroll
        for (int i = 0; i < WM; i++) {
          const u32x4 v = epi.pack(n0 + 16 * (wf * WN + j) + 4 * lq, acc[j][i]);
          *reinterpret_cast<u32x2*>(lds + base + (16 * i + lr) * RP + (16 * j + 4 * lq) / 4 * OB) = u32x2{v[0], v[1]};
        }
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0) alone (vmcnt 63, expcnt 7): this wave's rows are in LDS
      asm volatile("" ::: "memory");
      constexpr int TPR = RB / 16, RPP = 64 / TPR;  // lanes per row, rows per instruction
      const int tc = lane % TPR;
#pragma unroll 4
      for (int r = lane / TPR; r < WR; r += RPP) {
        const int m = m0 + WR * wt + r;
        if (m < g.M)
          st_b128(epi.ws, epi.row_off(m, n0 + 128 / FW * wf) + (uint32_t)(tc * 16), lds128(base + (uint32_t)(r * RP + tc * 16)));
      }
    }
    __syncthreads();  // the staged rows are read before the next tile's copies land
  } else {
  if (16 * tb0 >= g.M) return;
  if constexpr (HasPre<Epi>::value) {
    typename Epi::Pre pre[WN][WM];
#pragma unroll
    for (int j = 0; j < WN; j++)
#pragma unroll
      for (int i = 0; i < WM; i++) {
        const int m = m0 + 16 * (WM * wt + i) + lr;
        pre[j][i] = epi.pre(n0 + 16 * (wf * WN + j) + 4 * lq, m < g.M ? m : 0);
      }
#pragma unroll
    for (int j = 0; j < WN; j++)
#pragma unroll
      for (int i = 0; i < WM; i++) {
        const int m = m0 + 16 * (WM * wt + i) + lr;
        if (m < g.M) epi(n0 + 16 * (wf * WN + j) + 4 * lq, m, acc[j][i], pre[j][i]);
      }
  } else {
#pragma unroll
    for (int j = 0; j < WN; j++)
#pragma unroll
      for (int i = 0; i < WM; i++) {
        const int m = m0 + 16 * (WM * wt + i) + lr;
        if (m < g.M) epi(n0 + 16 * (wf * WN + j) + 4 * lq, m, acc[j][i]);
      }
  }
  }
}

// Every (16 WM TW) x 128 tile of an [M x N] GEMM (N a multiple of 128), K split into `ksplit` ranges
// (multiples of 128); items m-tile fastest, as in gemm_stage. The epilogue gets the split in epi.split.
template <int TW, int WM, class Epi>
__device__ __forceinline__ void gemm_stage_d(const GemmArgsF& g, int N, int K, int ksplit, Epi& epi) {
  constexpr int BM = 16 * WM * TW;
  const int nm = (g.M + BM - 1) / BM, nn = N / 128;
  const int items = nm * nn * ksplit, kc = K / ksplit;
#pragma unroll 1
  for (int it = vwg(); it < items; it += NWG) {
    const int mt = it % nm, rest = it / nm, nt = rest % nn, sp = rest / nn;
    epi.split = sp;
    gemm_tile_d<TW, WM>(g, mt * BM, nt * 128, sp * kc, sp * kc + kc, epi);
  }
}

template <class Epi>
__device__ __forceinline__ void gemm_stage_tall(const GemmArgsF& g, int N, int K, int ksplit, Epi& epi) {
  gemm_stage_d<NWAVE, 4>(g, N, K, ksplit, epi);
}

// Split-K GEMM whose K-splits are summed inside the stage (for small tiles: one workgroup reads the
// whole tile's partials, so large tiles leave the sum to the consumer stage instead): every split
// stores its fp32 partial
// [split][MP][N] (sc1), drains its stores, then bumps the tile's counter with a device-scope atomic.
// The workgroup that brings the count to ksplit resets it, reads the ksplit partials of the tile in
// split order (so the sum is deterministic) and hands fin(n, m, sum of columns n..n+3) for each of
// the tile's rows m < M. Consumers then read one finished value instead of ksplit partials.
// `counters` holds one zeroed word per output tile; `flag_lds` is an LDS word outside the GEMM ring.
constexpr int FIXUP_MAX_KS = 16;

template <int WM, int WN, bool AF = false, class Fin>
__device__ __forceinline__ void gemm_stage_fixup(const GemmArgs& g, int N, int K, int ksplit, rsrc_t ws,
                                                 uint32_t part_off, int MP, unsigned* counters, uint32_t flag_lds,
                                                 Fin& fin) {
  using S = GemmShape<WM, WN, AF>;
  struct Part : NoPre {
    rsrc_t ws;
    uint32_t off;
    int MP, N, split;
    __device__ void operator()(int n0, int m, f32x4 v, Pre) const {
      st_b128(ws, off + (uint32_t)((((size_t)split * MP + m) * N + n0) * 4), as_u32x4(v));
    }
  };
  struct Direct : NoPre {  // ksplit == 1: the tile's own result is final
    Fin* fin;
    int split;
    __device__ void operator()(int n0, int m, f32x4 v, Pre) const { (*fin)(n0, m, v); }
  };
  const int nm = (g.M + S::BM - 1) / S::BM, nn = N / S::BN;
  const int items = nm * nn * ksplit, kc = K / ksplit;
  if (ksplit == 1) {
    Direct d{{}, &fin, 0};
#pragma unroll 1
    for (int it = vwg(); it < items; it += NWG) {
      const int mt = it % nm, nt = it / nm;
      gemm_tile<WM, WN, AF>(g, mt * S::BM, nt * S::BN, 0, K, d);
    }
    return;
  }
  Part epi{{}, ws, part_off, MP, N, 0};
  unsigned* flag = reinterpret_cast<unsigned*>(lds + flag_lds);
  constexpr int Q = S::BN / 4;  // float4 columns per tile row
#pragma unroll 1
  for (int it = vwg(); it < items; it += NWG) {
    const int mt = it % nm, rest = it / nm, nt = rest % nn, sp = rest / nn;
    epi.split = sp;
    gemm_tile<WM, WN, AF>(g, mt * S::BM, nt * S::BN, sp * kc, sp * kc + kc, epi);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores are complete
    __syncthreads();
    if (threadIdx.x == 0) {
      unsigned* c = counters + mt * nn + nt;
      const unsigned old = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const unsigned last = old == (unsigned)ksplit - 1u;
      if (last) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      *flag = last;
    }
    __syncthreads();
    if (!*flag) continue;
#pragma unroll 1
    for (int e = tid(); e < S::BM * Q; e += NTHR) {
      const int m = mt * S::BM + e / Q, n = nt * S::BN + 4 * (e % Q);
      if (m >= g.M) continue;
      u32x4 v[FIXUP_MAX_KS];
#pragma unroll
      for (int s2 = 0; s2 < FIXUP_MAX_KS; s2++)
        if (s2 < ksplit) v[s2] = ldb128<kCpSc1>(ws, part_off + (uint32_t)((((size_t)s2 * MP + m) * N + n) * 4));
      f32x4 sum = as_f32x4(v[0]);
#pragma unroll
      for (int s2 = 1; s2 < FIXUP_MAX_KS; s2++)
        if (s2 < ksplit) sum += as_f32x4(v[s2]);
      fin(n, m, sum);
    }
  }
}

}  // namespace eng
}  // namespace fa
