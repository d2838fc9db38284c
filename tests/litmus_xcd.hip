// Litmus tests of the cross-CU message passing every kernel of the library relies on (MI355X, gfx950):
//   xcd  : data from one XCD to another: data stores with sc1 (write-through), s_waitcnt, a flag store
//          with sc1; the reader polls the flag with sc1 loads, then reads the data with sc1 loads.
//   local: data between two CUs of one XCD: plain stores (they stay in the XCD's L2), s_waitcnt, a
//          plain flag store; the reader polls and reads with sc1 loads (which bypass its L1).
//   tag  : the batch-1 exchange: no flag; each fp16 value carries the round's parity in its lowest
//          mantissa bit; the reader polls the data itself until every value carries the parity.
// Each launch runs ROUNDS rounds on 8 channels at once (one producer and one consumer workgroup per
// channel, on the XCDs the test names); a consumer stops at its first stale value and reports it.
// Every wait is capped, every index is in bounds, no value is used as an address.
// usage: litmus_xcd        prints one line per test and exits 0 when no read was stale.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int ROUNDS = 2000;
constexpr unsigned CAP = 1u << 20;  // polls per wait
constexpr int CH = 8;               // channels per launch
constexpr unsigned DATA = 1024;     // bytes of data per channel per round (one 16-byte slot per lane)
// buffer (bytes): data [CH][DATA] @0, flags [CH] one 128-byte line each @CH*DATA, the tag test's
// consumer acknowledgements [CH] one line each after them
constexpr unsigned FLAGS = CH * DATA, ACKS = FLAGS + CH * 128, BYTES = ACKS + CH * 128;

enum Mode { XCD = 0, LOCAL = 1, TAG = 2 };

__device__ __forceinline__ unsigned xcc() { return __builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 7u; }

// out[ch * 4 + 0..3] = stale reads, timeouts, first stale round (+1), placement errors
__global__ void __launch_bounds__(64) litmus(unsigned char* buf, int mode, int d, unsigned* out) {
  const int lane = threadIdx.x, x = blockIdx.x & 7, rk = blockIdx.x >> 3;
  const auto r = __builtin_amdgcn_make_buffer_rsrc(buf, (short)0, (int)BYTES, 0x00020000);
  // channel x: producer = rank 0 of XCD x; consumer = rank 0 of XCD (x + d) % 8 (xcd, tag) or rank 1
  // of XCD x (local)
  const bool prod = rk == 0;
  const bool cons = mode == LOCAL ? rk == 1 : rk == 0;
  if (!prod && !cons) return;
  if (lane == 0 && xcc() != (unsigned)x) atomicAdd(&out[x * 4 + 3], 1u);
  const int pch = x;                                     // channel this workgroup produces
  const int cch = mode == LOCAL ? x : (x - d + 8) % 8;   // channel this workgroup consumes
  bool stopped = false;
  for (unsigned i = 1; i <= ROUNDS; i++) {
    if (prod && !(mode == LOCAL && rk != 0)) {
      const unsigned doff = pch * DATA + lane * 16;
      if (mode == TAG) {
        // a value two rounds old carries this round's parity, so the producer waits until the
        // consumer has acknowledged round i - 1 before it overwrites it with round i
        for (unsigned it = 0; i > 1 && it < CAP; it++) {
          const unsigned a = __builtin_amdgcn_raw_buffer_load_b32(r, ACKS + pch * 128, 0, 16);
          if (__builtin_amdgcn_readfirstlane(a) >= i - 1) break;
          __builtin_amdgcn_s_sleep(1);
        }
        // eight fp16 values 1 + (i % 512) / 1024 with the lowest mantissa bit = i & 1
        const unsigned short h = (unsigned short)(0x3C00u | (((i % 512u) << 1) & 0x3FEu) | (i & 1u));
        const unsigned w = h | ((unsigned)h << 16);
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{w, w, w, w}, r, doff, 0, 16);
      } else {
        if (mode == LOCAL) {  // plain stores: the data stays in this XCD's L2
          __builtin_amdgcn_raw_buffer_store_b128(u32x4{i, i, i, i}, r, doff, 0, 0);
          __builtin_amdgcn_s_waitcnt(0);  // the data has reached L2
          if (lane == 0) __builtin_amdgcn_raw_buffer_store_b32(i, r, FLAGS + pch * 128, 0, 0);
        } else {  // sc1 stores: written through to memory
          __builtin_amdgcn_raw_buffer_store_b128(u32x4{i, i, i, i}, r, doff, 0, 16);
          __builtin_amdgcn_s_waitcnt(0);  // the data has reached memory
          if (lane == 0) __builtin_amdgcn_raw_buffer_store_b32(i, r, FLAGS + pch * 128, 0, 16);
        }
      }
    }
    if (cons && !stopped) {
      const unsigned doff = cch * DATA + lane * 16;
      unsigned it = 0;
      bool ok = false;
      if (mode == TAG) {
        const unsigned short h = (unsigned short)(0x3C00u | (((i % 512u) << 1) & 0x3FEu) | (i & 1u));
        const unsigned w = h | ((unsigned)h << 16);
        for (; it < CAP; it++) {
          const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, doff, 0, 16);
          const unsigned par = (i & 1u) * 0x00010001u;
          const bool cur = (((v[0] ^ par) | (v[1] ^ par) | (v[2] ^ par) | (v[3] ^ par)) & 0x00010001u) == 0;
          if (__builtin_amdgcn_ballot_w64(!cur) == 0) {
            // every value carries this round's parity: it must be this round's value (the producer
            // is at most one round ahead: it waits for this consumer's acknowledgement)
            ok = __builtin_amdgcn_ballot_w64(!(v[0] == w && v[1] == w && v[2] == w && v[3] == w)) == 0;
            break;
          }
          __builtin_amdgcn_s_sleep(1);
        }
      } else {
        for (; it < CAP; it++) {
          const unsigned f = __builtin_amdgcn_raw_buffer_load_b32(r, FLAGS + cch * 128, 0, 16);
          if (__builtin_amdgcn_readfirstlane(f) >= i) break;
          __builtin_amdgcn_s_sleep(1);
        }
        if (it < CAP) {
          const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, doff, 0, 16);
          // the producer may already be a round ahead (>= i); a value below i is stale
          ok = __builtin_amdgcn_ballot_w64(!(v[0] >= i && v[1] >= i && v[2] >= i && v[3] >= i)) == 0;
        }
      }
      if (it >= CAP) {
        if (lane == 0) atomicAdd(&out[cch * 4 + 1], 1u);
        stopped = true;
      } else if (!ok) {
        if (lane == 0) {
          atomicAdd(&out[cch * 4 + 0], 1u);
          atomicMax(&out[cch * 4 + 2], i);
        }
        stopped = true;  // stop at the first stale read
      }
    }
    // the tag test's acknowledgement (also after a stop, so the producer never waits out its cap)
    if (cons && mode == TAG && lane == 0) __builtin_amdgcn_raw_buffer_store_b32(i, r, ACKS + cch * 128, 0, 16);
  }
}

static int run(const char* name, int mode, int d) {
  unsigned char* buf = nullptr;
  unsigned* out = nullptr;
  if (hipMalloc(&buf, BYTES) != hipSuccess || hipMalloc(&out, CH * 4 * 4) != hipSuccess) return 2;
  if (hipMemset(buf, 0, BYTES) != hipSuccess || hipMemset(out, 0, CH * 4 * 4) != hipSuccess) return 2;
  hipLaunchKernelGGL(litmus, dim3(256), dim3(64), 0, 0, buf, mode, d, out);
  if (hipDeviceSynchronize() != hipSuccess) return 3;
  unsigned h[CH * 4];
  if (hipMemcpy(h, out, sizeof(h), hipMemcpyDeviceToHost) != hipSuccess) return 3;
  unsigned stale = 0, tmo = 0, first = 0, place = 0;
  for (int c = 0; c < CH; c++) {
    stale += h[c * 4];
    tmo += h[c * 4 + 1];
    if (h[c * 4 + 2] && (!first || h[c * 4 + 2] < first)) first = h[c * 4 + 2];
    place += h[c * 4 + 3];
  }
  printf("%-5s d=%d: %d rounds x %d channels, stale %u (first in round %u), timeouts %u, placement errors %u\n",
         name, d, ROUNDS, CH, stale, first, tmo, place);
  (void)hipFree(buf);
  (void)hipFree(out);
  return stale || tmo || place ? 1 : 0;
}

int main() {
  int bad = 0;
  bad |= run("local", LOCAL, 0);
  for (int d = 1; d < 8; d++) bad |= run("xcd", XCD, d);
  for (int d = 1; d < 8; d += 3) bad |= run("tag", TAG, d);
  printf(bad ? "LITMUS FAILED\n" : "LITMUS OK\n");
  return bad;
}
