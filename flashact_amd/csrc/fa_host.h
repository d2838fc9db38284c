// Host-side helpers shared by the C-ABI launchers: thread-local error text and the
// device / cooperative-capacity checks run before every launch.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/flashact_mi355x.h"

namespace fa {
namespace host {

char* error_buffer();  // thread-local, 512 bytes (capi.hip)

inline int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(error_buffer(), 512, fmt, ap);
  va_end(ap);
  return code;
}

// Enqueues the cooperative launch of `kernel` (nwg x threads, `lds` bytes of dynamic LDS). On failure
// the error text names the runtime's reason; hipErrorIllegalState is the refusal a process gets
// when its parent had already made a cooperative launch before starting it (measured: a child started
// before the parent's first cooperative launch launches normally), so the text says so.
int coop_launch(const void* kernel, int nwg, int threads, void** args, unsigned lds, fa_stream_t stream,
                const char* who);

// Verifies the current device is a 256-CU gfx950 with cooperative launch, raises the
// kernel's dynamic-LDS limit (once per device and kernel) and checks that `nwg`
// workgroups of `threads` threads can be co-resident.
int check_device(const void* kernel, int threads, unsigned lds_bytes, int nwg, const char* who);

}  // namespace host

// Batched pi0.5 launch (batch >= 2), dispatched from fa_pi05_denoise after the shared checks.
size_t pi05_batched_workspace_bytes(int batch, int Tv, int Lmax);
int pi05_denoise_batched(const fa_pi05_args* a, fa_stream_t stream);

// K/V hand-off (srows > 0): enqueues the de-interleave / transpose of kvsrc_k / kvsrc_v into the
// caches ahead of the denoise launch. Arguments are checked by fa_pi05_denoise.
int pi05_kv_handoff(const fa_pi05_args* a, fa_stream_t stream);

// fp16 caches (cache_dtype == FA_DTYPE_F16): both caches -> the bf16 shadow ahead of the loop, and the
// rows the loop (and a hand-off) wrote -> the caller's fp16 caches after it. Elements per cache.
size_t pi05_cache_elems(int batch, int num_layers, int Lmax);
int pi05_cache_import(const fa_pi05_args* a, fa_stream_t stream);
int pi05_cache_export(const fa_pi05_args* a, fa_stream_t stream);

// Co-resident workgroups of the batch-1 pi0.5 kernel on a device (0 if it cannot run there).
int pi05_bs1_coop_capacity(int device);

// Batch-1 MolmoAct2 launch (XCD-local layout), dispatched from fa_ma2_flow when eligible.
bool ma2_bs1_eligible(int batch, int Tv, int Lkmax);
size_t ma2_bs1_workspace_bytes();
int ma2_bs1_launch(const fa_ma2_args* a, fa_stream_t stream);

}  // namespace fa
