// Device-side building blocks shared by the MI355X (gfx950) denoise kernels.
//
// Memory-coherence model used by every kernel in this library (measured on MI355X):
//  * Each XCD (32 CUs) has a private L2. A CU's stores go write-through L1 -> its XCD's L2.
//  * Data exchanged between CUs of the SAME XCD: plain stores, device-scope (sc1) loads.
//    sc1 loads bypass L1 and see L2-resident data written by sibling CUs.
//  * Data exchanged ACROSS XCDs: sc1 stores (write-through to memory) and sc1 loads.
//  * Barriers are epoch flags, never RMW atomics: a workgroup publishes its epoch with one
//    store; waiters poll a flag line with one sc1 vector load per lane.
//      XCD barrier  : flag line in the XCD's L2 (~0.5 us).
//      grid barrier : XCD barrier, then each XCD's rank-0 workgroup publishes the epoch with an
//                     sc1 store to an 8-entry line that every workgroup polls.
//    No agent-scope L2 writeback/invalidate (buffer_wbl2 / buffer_inv) is issued anywhere: on
//    MI355X those cost ~4 us per barrier.
//  * Every wait is capped; a cap hit sets a sticky error bit that makes all later waits return
//    at once, so a broken launch always drains instead of hanging.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Cache-policy operand of gfx950 buffer instructions.
constexpr int kCpPlain = 0;
constexpr int kCpSc1 = 16;   // device scope: bypass L1, coherent across CUs/XCDs
constexpr int kRsrcWord3 = 0x00020000;

// Sticky error bits written into the workspace control block.
constexpr unsigned kErrSpin = 1u;   // a barrier wait hit its cap
constexpr unsigned kErrXcd = 2u;    // blockIdx -> XCD mapping differs from the assumed round robin
constexpr unsigned kErrRange = 4u;  // an exchanged fp16 partial sum exceeded the fp16 range
constexpr unsigned kSpinCap = 1u << 20;

// Workspace rules shared by every kernel of the library, so that one workspace may serve any mix
// of entry points and shapes:
//  * Bytes [0, kWsDataBase) hold only control words (u64 launch sequence @0, u32 error bits @8,
//    u32 exchange parity bases @12 and @16, u32 owner @kWsOwner), u64 epoch flags and the split-K
//    fixup counters. Every kernel keeps its data at kWsDataBase and above.
//  * Epoch flags derive from the launch sequence (epoch = seq << 32 + n), so a flag left by any
//    earlier launch lies below every epoch of the current one.
//  * Fixup counters are zero at rest (the last arriver resets its counter).
//  * Parity-tagged exchange data is not self-invalidating: its parity sequence is only valid while
//    the data area has been written by the same kernel since. The owner word names the kernel that
//    last used the workspace; a parity-exchange kernel that finds another owner clears its exchange
//    region and restarts its parity sequence before the first exchange.
constexpr uint32_t kWsOwner = 20;
constexpr uint32_t kWsCounters = 12288;  // [1024] u32
constexpr uint32_t kWsMaxCounters = 1024;
constexpr uint32_t kWsDataBase = 16384;
constexpr unsigned kOwnerPi05Bs1 = 1, kOwnerPi05Batched = 2, kOwnerMa2Bs1 = 3, kOwnerMa2Generic = 4,
                   kOwnerPrefill = 5;

__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, kRsrcWord3);
}

template <int CP>
__device__ __forceinline__ u32x4 ldb128(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, CP);
}
template <int CP>
__device__ __forceinline__ u32x2 ldb64(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, CP);
}
template <int CP>
__device__ __forceinline__ float ldbf32(rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, CP));
}
template <int CP>
__device__ __forceinline__ unsigned short ldb16(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, CP);
}
template <int CP>
__device__ __forceinline__ void stb128(rsrc_t r, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, CP);
}
template <int CP>
__device__ __forceinline__ void stb64(rsrc_t r, uint32_t off, u32x2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, CP);
}

// ---------------------------------------------------------------- parity-tagged fp16 exchange
// Cross-XCD partial sums travel as fp16 whose lowest mantissa bit carries the exchange parity, so
// data and flag are the same bits (see the batch-1 kernels). Rounding to nearest even (<= 0.5 ulp)
// and then forcing that bit (<= 1 ulp) leaves each value within 1.5 fp16 ulp of its fp32 sum, i.e.
// within 1.5 * 2^-10 relative for |v| >= 2^-14 and 1.5 * 2^-24 absolute below.
__device__ __forceinline__ unsigned pack_f16x2(float a, float b) {
  return (unsigned)__builtin_bit_cast(unsigned short, (_Float16)a) |
         ((unsigned)__builtin_bit_cast(unsigned short, (_Float16)b) << 16);
}
// |v| <= 65504 (the largest finite fp16); false for NaN as well.
__device__ __forceinline__ bool f16_finite(float v) { return fabsf(v) <= 65504.f; }
// Clamped to the finite fp16 range (NaN becomes 0), so the exchanged bits are never an infinity
// or a NaN, whose tagged forms would not be values at all.
__device__ __forceinline__ float f16_clamp(float v) { return f16_finite(v) ? v : (v > 0.f ? 65504.f : (v < 0.f ? -65504.f : 0.f)); }
// Four fp32 values -> four parity-tagged fp16 (8 bytes). `range` collects values outside the finite
// fp16 range (or NaN); those are exchanged clamped and the caller raises the sticky range status, so
// the launch's result is reported invalid instead of carrying an infinity into the residual stream.
__device__ __forceinline__ u32x2 tag16(f32x4 v, unsigned par, bool& range) {
  const unsigned pp = par * 0x00010001u;
  const bool ok = f16_finite(v[0]) && f16_finite(v[1]) && f16_finite(v[2]) && f16_finite(v[3]);
  range = range || !ok;
  if (!ok) v = f32x4{f16_clamp(v[0]), f16_clamp(v[1]), f16_clamp(v[2]), f16_clamp(v[3])};
  return u32x2{(pack_f16x2(v[0], v[1]) & ~0x00010001u) | pp, (pack_f16x2(v[2], v[3]) & ~0x00010001u) | pp};
}
// Non-zero if any of the eight fp16 of v carries the other parity.
__device__ __forceinline__ unsigned mism16(u32x4 v, unsigned par) {
  const unsigned pp = par * 0x00010001u;
  return ((v[0] ^ pp) | (v[1] ^ pp) | (v[2] ^ pp) | (v[3] ^ pp)) & 0x00010001u;
}
__device__ __forceinline__ float h_lo(unsigned u) { return (float)__builtin_bit_cast(_Float16, (unsigned short)(u & 0xffffu)); }
__device__ __forceinline__ float h_hi(unsigned u) { return (float)__builtin_bit_cast(_Float16, (unsigned short)(u >> 16)); }

__device__ __forceinline__ u32x4 ld_stream128(const void* p) {  // weights: read once per step
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  // D[16x16] += A[16x32] * B[32x16]. Lane l: A row l%16, B col l%16, k = 8*(l/16)..+7;
  // D rows 4*(l/16)+i, col l%16.
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0,
                                                 0, 0);
}

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
// The same product with fp16 operands (v_mfma_f32_16x16x32_f16, the bf16 rate on gfx950): the
// batch-1 attention on the caller's fp16 caches.
__device__ __forceinline__ f32x4 mfma16h(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                0);
}

// hipcc (ROCm 7.2, clang 22) evaluates __builtin_bit_cast(T, v[i]) on an element of an
// ext_vector_type as a cast of element 0. Element reinterpretation therefore goes through
// these value-parameter helpers; flashact_amd/build.py rejects the direct form in csrc/.
__device__ __forceinline__ float as_f32(unsigned u) { return __builtin_bit_cast(float, u); }
__device__ __forceinline__ unsigned as_u32(float f) { return __builtin_bit_cast(unsigned, f); }
__device__ __forceinline__ f32x4 as_f32x4(u32x4 u) { return __builtin_bit_cast(f32x4, u); }
__device__ __forceinline__ u32x4 as_u32x4(f32x4 f) { return __builtin_bit_cast(u32x4, f); }
__device__ __forceinline__ float bf2f(bf16 v) { return (float)v; }
__device__ __forceinline__ unsigned pack_bf16x2(float a, float b) {
  bf16x2 v = {(bf16)a, (bf16)b};
  return __builtin_bit_cast(unsigned, v);
}
__device__ __forceinline__ unsigned short bf16_bits(float a) { return __builtin_bit_cast(unsigned short, (bf16)a); }
__device__ __forceinline__ float bf_lo(unsigned u) { return __builtin_bit_cast(float, u << 16); }
__device__ __forceinline__ float bf_hi(unsigned u) { return __builtin_bit_cast(float, u & 0xffff0000u); }

__device__ __forceinline__ unsigned xcc_id() { return __builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 7u; }

// Cross-lane reductions without LDS round trips (lane layouts checked on gfx950 hardware):
//  * DPP inside a 16-lane row: quad_perm [1,0,3,2] (lane ^ 1), [2,3,0,1] (lane ^ 2),
//    row_half_mirror (i -> 7 - i in each half row), row_mirror (i -> 15 - i);
//  * v_permlane16_swap(x, y): lanes of even rows get {x own, x of lane + 16}, odd rows
//    {y of lane - 16, y own}, i.e. result[0] comes from the lower lane, result[1] from the upper;
//  * v_permlane32_swap: the same between the two 32-lane halves.
// Each combine applies the operator as (lower lane, upper lane), so every lane of a reduction
// group ends with the bit-identical value.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return as_f32((unsigned)__builtin_amdgcn_update_dpp(0, (int)as_u32(v), CTRL, 0xF, 0xF, false));
}
// lane l gets the value of lane l ^ 1 (DPP quad_perm [1, 0, 3, 2])
__device__ __forceinline__ unsigned swap_adj(unsigned v) {
  return (unsigned)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xF, 0xF, false);
}
struct LanePair {
  unsigned lo, hi;
};
__device__ __forceinline__ LanePair swap16(unsigned x, unsigned y) {
  const auto r = __builtin_amdgcn_permlane16_swap(x, y, false, false);
  return {r[0], r[1]};
}
__device__ __forceinline__ LanePair swap32(unsigned x, unsigned y) {
  const auto r = __builtin_amdgcn_permlane32_swap(x, y, false, false);
  return {r[0], r[1]};
}
// Sum / max over the lanes {l, l ^ 16, l ^ 32, l ^ 48} (the four row-quarters of a column).
__device__ __forceinline__ float cols_sum(float v) {
  LanePair a = swap16(as_u32(v), as_u32(v));
  v = as_f32(a.lo) + as_f32(a.hi);
  a = swap32(as_u32(v), as_u32(v));
  return as_f32(a.lo) + as_f32(a.hi);
}
__device__ __forceinline__ float cols_max(float v) {
  LanePair a = swap16(as_u32(v), as_u32(v));
  v = fmaxf(as_f32(a.lo), as_f32(a.hi));
  a = swap32(as_u32(v), as_u32(v));
  return fmaxf(as_f32(a.lo), as_f32(a.hi));
}
// Value of lane ^ 16 (selected from the swap of x with itself).
__device__ __forceinline__ unsigned xor16_u32(unsigned x, bool odd_row) {
  const LanePair a = swap16(x, x);
  return odd_row ? a.lo : a.hi;
}
__device__ __forceinline__ float wave_sum(float v) {
  v = dpp_f32<0xB1>(v) + v;
  v = dpp_f32<0x4E>(v) + v;
  v = dpp_f32<0x141>(v) + v;
  v = dpp_f32<0x140>(v) + v;
  return cols_sum(v);
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(dpp_f32<0xB1>(v), v);
  v = fmaxf(dpp_f32<0x4E>(v), v);
  v = fmaxf(dpp_f32<0x141>(v), v);
  v = fmaxf(dpp_f32<0x140>(v), v);
  return cols_max(v);
}

// GeLU with the tanh approximation (Hendrycks & Gimpel 2016), x (1 + tanh y) / 2 with
// y = sqrt(2/pi) (x + 0.044715 x^3), written through the identity (1 + tanh y) / 2 = 1 / (1 + e^-2y)
// as x / (1 + 2^(-2 y log2 e)): one v_exp_f32 and one v_rcp_f32 (about 1 ulp each) and five more
// instructions, where tanhf took about 30 with both of its branches. The tails need no care:
// 2^t -> inf gives x * 0, 2^t -> 0 gives x. (Prefill 6.54 -> 6.18 ms, pi0.5 batch 16 21.5 -> 21.2 ms.)
__device__ __forceinline__ float gelu_tanh(float x) {
  constexpr float c1 = -2.0f * 0.7978845608028654f * 1.4426950408889634f;  // -2 sqrt(2/pi) log2(e)
  constexpr float c3 = c1 * 0.044715f;
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * (c1 + c3 * (x * x))));
}
// x / (1 + e^-x) in the same form (expf and an IEEE divide took about 25 instructions).
__device__ __forceinline__ float silu(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

// 2^x as the bare v_exp_f32, for softmax weights and their rescale factors: a result below 2^-126
// comes out as zero or a flushed value instead of an exact denormal (exp2f adds a range fix-up of
// four more instructions per call for that case). Weights that small vanish against the row sum.
__device__ __forceinline__ float exp2_w(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------- barriers
struct Sync {
  uint64_t* xline;  // this XCD's flag line, one slot per rank
  uint64_t* gline;  // one slot per XCD
  unsigned* err;
  uint64_t e;       // epoch of the most recent arrive
  int rank, xcd, nrank, nxcd;
};

__device__ __forceinline__ uint64_t ld_flag(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One full wave polls p[0..n) until every entry >= e.
__device__ __forceinline__ void poll_wave(const uint64_t* p, int n, uint64_t e, unsigned* err) {
  if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & kErrSpin) return;
  const int lane = threadIdx.x & 63;
  for (unsigned it = 0;; ++it) {
    uint64_t v = lane < n ? ld_flag(p + lane) : ~0ull;
    if (__all(v >= e)) return;
    if (it > kSpinCap) {
      if (lane == 0) atomicOr(err, kErrSpin);
      return;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// One full wave polls the u64 epoch flags at [off, off + bytes) of `ws` (bytes a multiple of
// 1024) until every flag >= e; 16 bytes per lane and 1 KB per sc1 load round.
__device__ __forceinline__ void poll_flags(rsrc_t ws, uint32_t off, uint32_t bytes, uint64_t e, unsigned* err) {
  if (__hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & kErrSpin) return;
  const int lane = threadIdx.x & 63;
  for (unsigned it = 0;; ++it) {
    bool ok = true;
    for (uint32_t o = 16u * lane; o < bytes; o += 1024u) {
      const u32x4 v = ldb128<kCpSc1>(ws, off + o);
      ok = ok && ((((uint64_t)v[1] << 32) | v[0]) >= e) && ((((uint64_t)v[3] << 32) | v[2]) >= e);
    }
    if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
    if (it > kSpinCap) {
      if (lane == 0) atomicOr(err, kErrSpin);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  asm volatile("" ::: "memory");
}

// Publish this workgroup's epoch. All of the workgroup's prior global stores are complete
// (vmcnt drained) before the flag store issues.
__device__ __forceinline__ void sync_arrive(Sync& s) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  s.e += 1;
  if (threadIdx.x == 0) __hip_atomic_store(&s.xline[s.rank], s.e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ void sync_wait_xcd(Sync& s) {
  if (threadIdx.x < 64) poll_wave(s.xline, s.nrank, s.e, s.err);
  __syncthreads();
}

__device__ __forceinline__ void sync_wait_grid(Sync& s) {
  if (threadIdx.x < 64) {
    if (s.rank == 0) {
      poll_wave(s.xline, s.nrank, s.e, s.err);
      if (threadIdx.x == 0) __hip_atomic_store(&s.gline[s.xcd], s.e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    poll_wave(s.gline, s.nxcd, s.e, s.err);
  }
  __syncthreads();
}

}  // namespace fa
