// Latency and bandwidth probe of the MI355X fabric (gfx950), the measurements behind the per-phase
// latency budget of the batch-1 kernels:
//   handoff: one wave of workgroup 0 and one wave of a partner workgroup pass a round number back and
//            forth ROUNDS times. Workgroup 0 stores 1 KB of data, waits for the stores (timed: the
//            store acknowledgement), stores a flag; the partner polls the flag (sc1 loads), reads and
//            checks the data (sc1), stores its own flag; workgroup 0 polls that (the whole round trip is
//            timed). Partner 8 (rank 1 of XCD 0) is on workgroup 0's XCD: data and flags as plain stores,
//            which stay in the XCD's L2, or as sc1 stores. Partner 1 is on XCD 1: sc1 stores (plain
//            stores would stay in XCD 0's L2 and never reach it).
//   stream : 256 workgroups read a 1 GiB buffer in 32 MiB chunks (each XCD's 32 CUs split a chunk), in
//            three modes: every XCD reads the same chunk sequence; every XCD reads its own chunks; XCD 0
//            alone. Bandwidth per XCD and over the active XCDs.
// Every index is in bounds, every wait is capped (a side whose wait hits the cap stops), and only
// workgroups 0 and the partner take part in a hand-off (the others return at once); the stream kernel
// stores one word per workgroup at most.
// usage: fabric_probe      prints one line per measurement, then "FABRIC OK" when no read was stale,
//                          no wait hit its cap and every workgroup ran on the XCD its index implies.
#include <hip/hip_runtime.h>

#include <cstdio>

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int ROUNDS = 400;
constexpr unsigned CAP = 1u << 20;                 // polls per wait
constexpr unsigned DATA = 64 * 1024;               // data ring: 64 slots of 1 KB
constexpr unsigned F0 = DATA, F1 = DATA + 4096;    // flags, one per side, 4 KB apart
constexpr unsigned BUF = DATA + 8192;

__device__ __forceinline__ unsigned xcc() { return __builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 7u; }

// out[0] store-ack ticks, [1] round-trip ticks (100 MHz ticks, summed over rounds), [3] stale reads,
// [4] / [7] capped waits of workgroup 0 / the partner, [5] XCD of workgroup 0, [6] XCD of the partner
template <int CP>
__global__ void __launch_bounds__(64) handoff(unsigned char* buf, int partner, unsigned long long* out) {
  const int me = blockIdx.x, lane = threadIdx.x;
  if (me != 0 && me != partner) return;
  const auto r = __builtin_amdgcn_make_buffer_rsrc(buf, (short)0, (int)BUF, 0x00020000);
  unsigned long long ack = 0, rt = 0, bad = 0, capped = 0;
  if (lane == 0) out[me == 0 ? 5 : 6] = xcc();
  for (unsigned i = 1; i <= ROUNDS; i++) {
    const unsigned doff = (i % 64) * 1024 + lane * 16;
    if (me == 0) {
      const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{i, i, i, i}, r, doff, 0, CP);
      __builtin_amdgcn_s_waitcnt(0);
      const unsigned long long t1 = __builtin_amdgcn_s_memrealtime();
      if (lane == 0) __builtin_amdgcn_raw_buffer_store_b32(i, r, F0, 0, CP);
      unsigned it = 0;
      for (; it < CAP; it++) {
        if (__builtin_amdgcn_readfirstlane(__builtin_amdgcn_raw_buffer_load_b32(r, F1, 0, 16)) == i) break;
        __builtin_amdgcn_s_sleep(1);
      }
      const unsigned long long t2 = __builtin_amdgcn_s_memrealtime();
      ack += t1 - t0;
      rt += t2 - t0;
      if (it >= CAP) {  // the partner is gone: stop (it stops at its own next capped wait)
        capped++;
        break;
      }
    } else {
      unsigned it = 0;
      for (; it < CAP; it++) {
        if (__builtin_amdgcn_readfirstlane(__builtin_amdgcn_raw_buffer_load_b32(r, F0, 0, 16)) == i) break;
        __builtin_amdgcn_s_sleep(1);
      }
      if (it >= CAP) {
        capped++;
        break;
      }
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, doff, 0, 16);
      bad += (v[0] != i) | (v[3] != i);
      if (lane == 0) __builtin_amdgcn_raw_buffer_store_b32(i, r, F1, 0, CP);
      __builtin_amdgcn_s_waitcnt(0);
    }
  }
  // stale reads and capped waits of any lane; timings of lane 0
  bad = __builtin_amdgcn_ballot_w64(bad != 0) != 0;
  if (lane == 0) {
    if (me == 0) {
      out[0] = ack;
      out[1] = rt;
      out[4] = capped;
    } else {
      out[3] = bad;
      out[7] = capped;
    }
  }
}

// Workgroup b runs on XCD b % 8 as rank b / 8 (recorded in xccs). mode 0: every XCD reads the same
// chunk sequence; mode 1: each XCD its own chunks; mode 2: XCD 0 alone.
__global__ void __launch_bounds__(256) stream(const unsigned char* W, unsigned long long size, int mode, int chunks,
                                              unsigned long long cb, unsigned* sink, unsigned* xccs) {
  const int x = blockIdx.x & 7, rk = blockIdx.x >> 3;
  if (threadIdx.x == 0) xccs[blockIdx.x] = xcc();
  if (mode == 2 && x != 0) return;
  u32x4 acc = {0, 0, 0, 0};
  const unsigned long long per_cu = cb / 32;  // bytes of a chunk per CU
  for (int c = 0; c < chunks; c++) {
    const unsigned long long base =
        mode == 1 ? ((unsigned long long)(c * 8 + x) * cb) % size : ((unsigned long long)c * cb) % size;
    const unsigned char* p = W + base + rk * per_cu;
    for (unsigned long long o = threadIdx.x * 16; o < per_cu; o += 256 * 16 * 8) {
      u32x4 v[8];
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const unsigned long long oo = o + k * 256 * 16;
        v[k] = oo < per_cu ? *reinterpret_cast<const u32x4*>(p + oo) : u32x4{0, 0, 0, 0};
      }
#pragma unroll
      for (int k = 0; k < 8; k++) acc ^= v[k];
    }
  }
  const unsigned s = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (s == 0x12345678u) sink[blockIdx.x] = s;  // keeps the loads live
}

int main() {
  unsigned char* buf = nullptr;
  unsigned long long* out = nullptr;
  if (hipMalloc(&buf, BUF) != hipSuccess || hipMalloc(&out, 8 * 8) != hipSuccess) return 2;
  int bad = 0;
  const int cases[3][2] = {{8, 0}, {8, 1}, {1, 1}};  // (partner, sc1 stores)
  for (const auto& cs : cases) {
    const int partner = cs[0], sc1 = cs[1];
    {
      if (hipMemset(buf, 0, BUF) != hipSuccess || hipMemset(out, 0, 64) != hipSuccess) return 2;
      if (sc1)
        hipLaunchKernelGGL(handoff<16>, dim3(256), dim3(64), 0, 0, buf, partner, out);
      else
        hipLaunchKernelGGL(handoff<0>, dim3(256), dim3(64), 0, 0, buf, partner, out);
      if (hipDeviceSynchronize() != hipSuccess) return 3;
      unsigned long long t[8];
      if (hipMemcpy(t, out, sizeof(t), hipMemcpyDeviceToHost) != hipSuccess) return 3;
      const bool same = t[5] == t[6];
      if (t[5] != 0 || t[6] != (unsigned long long)(partner % 8)) bad = 1;
      if (t[3] || t[4] || t[7]) bad = 1;
      printf("handoff %s %s: store_ack_ns %.0f round_trip_ns %.0f stale %llu capped %llu\n", same ? "same-xcd" : "cross-xcd",
             sc1 ? "sc1" : "plain", t[0] * 10.0 / ROUNDS, t[1] * 10.0 / ROUNDS, t[3], t[4] + t[7]);
    }
  }
  (void)hipFree(buf);
  (void)hipFree(out);

  const unsigned long long size = 1ull << 30, cb = 32ull << 20;
  unsigned char* W = nullptr;
  unsigned *sink = nullptr, *xccs = nullptr;
  if (hipMalloc(&W, size) != hipSuccess || hipMalloc(&sink, 4096) != hipSuccess || hipMalloc(&xccs, 4096) != hipSuccess)
    return 2;
  if (hipMemset(W, 7, size) != hipSuccess) return 2;
  hipEvent_t a, b;
  if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) return 2;
  const int chunks = (int)((2ull << 30) / cb / 8);  // 256 MiB per XCD
  const char* names[3] = {"same-data", "own-data", "xcd0-alone"};
  for (int mode = 0; mode < 3; mode++) {
    float ms = 0.f;
    for (int rep = 0; rep < 2; rep++) {  // the second launch is reported
      (void)hipEventRecord(a);
      hipLaunchKernelGGL(stream, dim3(256), dim3(256), 0, 0, W, size, mode, chunks, cb, sink, xccs);
      (void)hipEventRecord(b);
      if (hipEventSynchronize(b) != hipSuccess) return 3;
      (void)hipEventElapsedTime(&ms, a, b);
    }
    const double per_xcd = (double)chunks * cb;
    const int nx = mode == 2 ? 1 : 8;
    printf("stream %s: per_xcd_GBs %.0f total_GBs %.0f ms %.3f\n", names[mode], per_xcd / ms / 1e6,
           nx * per_xcd / ms / 1e6, ms);
  }
  unsigned h[256];
  if (hipMemcpy(h, xccs, sizeof(h), hipMemcpyDeviceToHost) != hipSuccess) return 3;
  for (int i = 0; i < 256; i++)
    if (h[i] != (unsigned)(i % 8)) bad = 1;
  (void)hipFree(W);
  (void)hipFree(sink);
  (void)hipFree(xccs);
  printf(bad ? "FABRIC FAILED\n" : "FABRIC OK\n");
  return bad;
}
