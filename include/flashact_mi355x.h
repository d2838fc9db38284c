/*
 * flashact_mi355x.h -- C ABI of the MI355X (gfx950) flow-matching denoise engine.
 *
 * Plain C: pointers, sizes and ints only. Every device pointer is HIP device memory owned
 * by the caller; no entry point allocates, frees or synchronises. Work is enqueued on the
 * given stream (a hipStream_t; NULL = the default stream). Entry points return FA_OK (0) or
 * an FA_ERR_* code; fa_last_error() returns the message of the calling thread's last failure.
 *
 * Reference interfaces replaced (paths relative to the FlashAct source tree):
 *   fa_pi05_denoise ....... `launch(...)` of the mk_v6 torch extension, src/pi05/binding.cpp:28-68
 *                            (kernel pi05_megakernel, src/pi05/mk6.cu:112-519)
 *   fa_ma2_flow ........... `launch(...)` of the mk_ma2 torch extension, src/molmoact2/binding.cpp:28-83
 *                            (kernel ma2_megakernel, src/molmoact2/mk_ma2.cu:103-576)
 *   fa_pi05_prefill ....... the prefix prefill (openpi PaliGemma forward with use_cache,
 *                            benchmarks/pi05/eval_numerics.py:50-57) and the K/V cache hand-off
 *                            after it (src/pi05/pack_weights.py:60-70, eval_numerics.py:83-87)
 *   fa_*_workspace_bytes,
 *   fa_*_workspace_init ... the reference's caller-allocated scratch tensors
 *                            (src/pi05/binding.cpp:34-36, src/molmoact2/binding.cpp:33-34)
 *   fa_last_error ......... TORCH_CHECK on the launch status (src/pi05/binding.cpp:67)
 *   fa_device_query ....... the occupancy clamp / diagnostics of src/molmoact2/binding.cpp:65-79
 *   fa_abi_version ........ no counterpart (ABI guard for the Python and C++ callers)
 */
#ifndef FLASHACT_MI355X_H
#define FLASHACT_MI355X_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FA_ABI_VERSION 2

/* Unit of every stage_cycles counter: ticks of the GPU's constant 100 MHz real-time clock
 * (s_memrealtime), accumulated (+=) into the caller's counters like the reference's clock64()
 * cycles (src/pi05/mk6.cu:129-134); the caller zeroes them. microseconds = ticks / 100. */
#define FA_STAGE_TICK_HZ 100000000

struct ihipStream_t;
typedef struct ihipStream_t* fa_stream_t; /* identical to hipStream_t */

enum fa_status {
  FA_OK = 0,
  FA_ERR_INVALID_ARG = 1,  /* bad shape, null or misaligned pointer, workspace too small */
  FA_ERR_UNSUPPORTED = 2,  /* valid request this build does not implement (e.g. fp8 weights) */
  FA_ERR_DEVICE = 3,       /* not a 256-CU gfx950, or cooperative launch unavailable */
  FA_ERR_LAUNCH = 4        /* the HIP launch itself failed */
};

enum fa_dtype { FA_DTYPE_BF16 = 0, FA_DTYPE_FP8_E4M3 = 1, FA_DTYPE_F16 = 2 };

/* Kernel-side status bits (read back from the workspace by fa_*_read_status). */
#define FA_KSTATUS_SPIN_TIMEOUT 1u /* a grid/XCD barrier wait hit its cap: results invalid */
#define FA_KSTATUS_XCD_MAP 2u      /* workgroup -> XCD placement differed from round robin */
#define FA_KSTATUS_RANGE 4u        /* a partial sum exchanged between XCDs left the finite fp16
                                    * range (|v| > 65504, or NaN) in the pi0.5 batch-1 kernel; it was
                                    * exchanged clamped to +-65504: results invalid */

typedef struct fa_device_info {
  int cus;               /* compute units */
  int xcds;              /* accelerator complex dies */
  int lds_bytes;         /* LDS per workgroup */
  int coop_launch;       /* cooperative launch supported */
  int coop_max_blocks;   /* co-resident workgroups of the batch-1 pi0.5 kernel (occupancy x CUs;
                          * 0 if that kernel cannot run on the device) */
  char arch[64];         /* gcnArchName */
} fa_device_info;

/* ---------------------------------------------------------------- pi0.5 expert
 * D=1024, 8 query heads / 1 KV head, head_dim 256, F=4096, action dim 32.
 * Weight packing is the reference's (src/pi05/hybrid_model.py:94-110):
 *   w1 [NL][2560][1024]: rows 2p, 2p+1 = q rows (h*256+j, h*256+j+128), p = h*128+j;
 *                        rows 2048+2j, 2048+2j+1 = k rows (j, j+128); rows 2304.. = v rows.
 *   wo [NL][1024][2048]; w2 [NL][8192][1024]: rows 2f = gate f, 2f+1 = up f; w3 [NL][1024][4096].
 * mods [S][NL][2][3072] (scale | shift | gate, for input/post-attention norms), mod_final [S][3072].
 * rope_cos/sin [Tv][128] for positions Lp + t. w_ain [1024][32], b_ain [1024], w_aout [32][1024],
 * b_aout [32] (fp32). kcache [batch][NL][Lmax][256] holds RoPE'd prefix keys in rows [0, Lp);
 * vtcache [batch][NL][256][Lmax] holds the transposed prefix values in columns [0, Lp). The caches
 * are bf16, or fp16 as the reference allocates them (benchmarks/pi05/eval_numerics.py:83-85,
 * src/pi05/hybrid_model.py:172-173): see cache_dtype.
 * The launch writes the suffix rows/columns [Lp, Lp+Tv) of both caches (as the reference does)
 * and updates x_t in place: x_t [batch][xt_rows][32] fp32, rows [0, Tv) of each sample.
 */
typedef struct fa_pi05_args {
  int weight_dtype; /* FA_DTYPE_BF16, or FA_DTYPE_FP8_E4M3 (batch 1): e4m3 codes in the same packed
                     * layouts with one fp32 scale per packed row in s1 [NL][2560], so [NL][1024],
                     * s2 [NL][8192], s3 [NL][1024] (src/pi05/hybrid_model.py:105-110) */
  const void* w1;
  const void* wo;
  const void* w2;
  const void* w3;
  const float* s1; /* per-row fp8 scales (16-byte aligned); must be NULL for bf16 weights */
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
  /* K/V hand-off (src/pi05/mk6.cu:258-277), used when srows > 0: kvsrc_k / kvsrc_v bf16
   * [batch][NL][srows][256] hold a prefill's cache rows with RoPE on interleaved pairs (2d, 2d+1).
   * Before the loop, rows [0, Lp) become kcache rows (pair -> dims d, d+128) and vtcache columns
   * (transposed); srows >= Lp. This runs as a separate kernel ahead of the loop on the same stream.
   * srows == 0: kcache / vtcache already hold the prefix and kvsrc_* are ignored. */
  const void* kvsrc_k;
  const void* kvsrc_v;
  int srows;
  void* kcache;
  void* vtcache;
  int Lp;
  int Lmax;
  int num_steps;
  int Tv;
  int num_layers; /* 18 for pi0.5 */
  int batch;      /* 1 (batched launches: see fa_pi05_max_batch) */
  float* x_t;
  int xt_rows;
  unsigned long long* stage_cycles; /* optional [16]: per-stage ticks (FA_STAGE_TICK_HZ), workgroup 0, += */
  void* workspace;
  size_t workspace_bytes;
  /* Diagnostics (optional): for global layer index trace_layer (= step * num_layers + layer),
   * every compute wave writes the 100 MHz real-time clock at the start and end of each stage of
   * that layer and at sub-stage points, and the first loader wave records when each of the
   * layer's weight pages was issued and landed: trace [256 workgroups][6][32]. NULL disables. */
  unsigned long long* trace;
  int trace_layer;
  /* Cache element type: FA_DTYPE_BF16 (0), or FA_DTYPE_F16 for the reference's fp16 caches.
   * fp16 caches at batch 1 with srows == 0 (the reference's own call): the loop reads and writes
   * them directly and runs its attention in fp16 (q, this step's keys and values, the softmax weights
   * and the cached keys and values as fp16 MFMA operands, as src/pi05/mk6.cu computes it);
   * cache_shadow is then not used and may be NULL.
   * fp16 caches otherwise (batch >= 2, or a hand-off with srows > 0): the launch converts both
   * caches to bf16 into cache_shadow (at least fa_pi05_cache_shadow_bytes(batch, num_layers, Lmax)
   * bytes, 256-byte aligned, caller-owned), runs the loop on the shadow (the hand-off writes it too)
   * and converts the rows it wrote back into the caller's fp16 caches: [Lp, Lp+Tv), and [0, Lp) as
   * well with srows > 0; fp16 -> bf16 rounds each cached value to 8 significant bits, as the bf16
   * operands of the attention MFMAs would. cache_shadow is ignored for bf16 caches. */
  int cache_dtype;
  void* cache_shadow;
  size_t cache_shadow_bytes;
} fa_pi05_args;

/* Whole S-step Euler loop as ONE cooperative launch (256 workgroups, one per CU). */
int fa_pi05_denoise(const fa_pi05_args* args, fa_stream_t stream);
size_t fa_pi05_workspace_bytes(int batch, int Tv, int Lmax);
/* fa_pi05_denoise without a caller workspace. No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). args->workspace must be NULL and workspace_bytes 0; the launch uses a
 * 16 MiB scratch the library reserves in device memory at load time (one per device, held until
 * the process ends), zeroed by a fill kernel on `stream` at the first call on each device.
 * Requests whose workspace (fa_pi05_workspace_bytes) exceeds 16 MiB are rejected
 * (FA_ERR_INVALID_ARG); every batch-1 request fits. No hipMalloc, hipFree or other allocating call
 * is made. All calls on one device share the scratch, which keeps the last call's contents: calls
 * that overlap on one GPU race (serialise them on one stream, or use fa_pi05_denoise with one
 * workspace per concurrent call). *scratch_out (optional) receives the scratch's device address,
 * for fa_pi05_read_status and fa_pi05_workspace_init. */
int fa_pi05_denoise_noalloc(const fa_pi05_args* args, fa_stream_t stream, void** scratch_out);
/* Bytes of the bf16 cache shadow an fp16-cache launch needs (see cache_dtype). */
size_t fa_pi05_cache_shadow_bytes(int batch, int num_layers, int Lmax);
/* Zeroes a workspace (required once after allocation and after a non-zero kernel status). */
int fa_pi05_workspace_init(void* workspace, size_t bytes, fa_stream_t stream);
/* Synchronous: copies the kernel status bits (FA_KSTATUS_*) of the last launch on this workspace. */
int fa_pi05_read_status(const void* workspace, unsigned* status);
/* Largest batch one launch accepts. batch 1 runs the latency-bound single-sample kernel, batch >= 2
 * the batched (MFMA-bound) kernel. The workspace size depends on the shape; one workspace that is
 * large enough may serve any sequence of launches of every entry point (never two at once). */
int fa_pi05_max_batch(void);

/* ---------------------------------------------------------------- MolmoAct2 expert
 * D=768, 8 heads of 96 (self attention over the action tokens, cross attention over the
 * context), F=3072, action dim 32 of which the first `adim` are integrated; t_s = s/S, dt = +1/S.
 * Weight packing is the reference's (benchmarks/molmoact2/eval_numerics.py:77-133), bf16:
 *   w_qkv [NL][2304][768] (q | k | v rows), w_so / w_cq / w_co [NL][768][768],
 *   w_gu [NL][6144][768] (rows 2f, 2f+1 = gate f, up f), w_dn [NL][768][3072]; w_aout [32][768].
 * Biases fp32: b_qkv [NL][2304], b_so / b_cq / b_co / b_dn [NL][768], b_gu [NL][6144] (interleaved
 * like w_gu), b_aout [32]; w_ain [768][32] and b_ain [768] fp32.
 * mods [S][NL][3][3][768] ({self, cross, mlp} x {scale, shift, gate}), mod_final [S][2][768]
 * (scale, shift). rope_cos/sin [Tv][48] for positions 0..Tv-1 (split-half pairs d, d+48).
 * kctx bf16 [batch][NL][Lkmax][768] (rows [0, Lk) valid), vtctx bf16 [batch][NL][768][Lkmax]
 * (columns [0, Lk) valid). x_t [batch][xt_rows][32] fp32 is updated in place for rows [0, Tv),
 * dims [0, adim).
 */
typedef struct fa_ma2_args {
  int weight_dtype; /* FA_DTYPE_BF16 */
  const void* w_qkv;
  const void* w_so;
  const void* w_cq;
  const void* w_co;
  const void* w_gu;
  const void* w_dn;
  const float* b_qkv;
  const float* b_so;
  const float* b_cq;
  const float* b_co;
  const float* b_gu;
  const float* b_dn;
  const float* mods;
  const float* mod_final;
  const float* rope_cos;
  const float* rope_sin;
  const float* w_ain;
  const float* b_ain;
  const void* w_aout;
  const float* b_aout;
  const void* kctx;
  const void* vtctx;
  int Lk;
  int Lkmax;
  int Tv;
  int adim;
  int num_steps;
  int num_layers; /* 36 for MolmoAct2 */
  int batch;
  float* x_t;
  int xt_rows;
  unsigned long long* stage_cycles; /* optional [16]: per-stage ticks (FA_STAGE_TICK_HZ), workgroup 0, += */
  void* workspace;
  size_t workspace_bytes;
} fa_ma2_args;

/* Whole S-step flow loop for `batch` samples as ONE cooperative launch (256 workgroups). */
int fa_ma2_flow(const fa_ma2_args* args, fa_stream_t stream);
size_t fa_ma2_workspace_bytes(int batch, int Tv, int Lkmax);
int fa_ma2_workspace_init(void* workspace, size_t bytes, fa_stream_t stream);
int fa_ma2_read_status(const void* workspace, unsigned* status);
int fa_ma2_max_batch(void);

/* ---------------------------------------------------------------- pi0.5 prefix prefill
 * The Gemma-2B-shaped backbone over the prefix (the benchmark's prefill workload): D=2048, 8 query heads / 1 KV
 * head of 256, F=16384 GeLU-tanh-gated MLP, RMSNorm (eps 1e-6) scaled by (1 + w), RoPE (base
 * 10000, split-half pairs j, j+128) at positions 0..Lp-1, bidirectional attention over the prefix.
 * Replaces the reference's prefix prefill, openpi's PaliGemma forward with use_cache
 * (benchmarks/pi05/eval_numerics.py:50-57), together with the cache hand-off after it (compact_kv,
 * src/pi05/pack_weights.py:60-70, and the cache fill at benchmarks/pi05/eval_numerics.py:83-87):
 * the launch writes the RoPE'd keys into kcache rows [0, Lp) and the transposed values into
 * vtcache columns [0, Lp) of every layer, the layout fa_pi05_denoise reads.
 * Weights bf16, packed like the expert's: wqkv [NL][2560][2048] (q/k RoPE pairs adjacent),
 * wo [NL][2048][2048], wgu [NL][32768][2048] (rows 2f, 2f+1 = gate f, up f), wdn [NL][2048][16384].
 * ln_in, ln_post [NL][2048] fp32: the input and post-attention RMSNorm weights of each layer.
 * rope_cos/sin [Lp][128]. x [batch][Lp][2048] fp32: the hidden states entering layer 0 (the
 * prefix embeddings after any embedding scaling). kcache [batch][NL][Lmax][256] and vtcache
 * [batch][NL][256][Lmax] bf16, Lmax >= Lp. Of the last layer only the K/V projections run: its
 * attention and MLP outputs reach no cache entry.
 * The workspace is zeroed with fa_pi05_workspace_init and read with fa_pi05_read_status.
 */
typedef struct fa_prefill_args {
  int weight_dtype; /* FA_DTYPE_BF16 */
  const void* wqkv;
  const void* wo;
  const void* wgu;
  const void* wdn;
  const float* ln_in;
  const float* ln_post;
  const float* rope_cos;
  const float* rope_sin;
  const float* x;
  void* kcache;
  void* vtcache;
  int Lp;
  int Lmax;
  int num_layers;
  int batch;
  unsigned long long* stage_cycles; /* optional [16]: per-stage ticks (FA_STAGE_TICK_HZ), workgroup 0, += */
  void* workspace;
  size_t workspace_bytes;
} fa_prefill_args;

/* All layers of the prefix prefill as ONE cooperative launch (256 workgroups). */
int fa_pi05_prefill(const fa_prefill_args* args, fa_stream_t stream);
size_t fa_pi05_prefill_workspace_bytes(int batch, int Lp, int Lmax);

/* ---------------------------------------------------------------- common */
int fa_device_query(int device, fa_device_info* info);
const char* fa_last_error(void);
int fa_abi_version(void);

#ifdef __cplusplus
}
#endif
#endif /* FLASHACT_MI355X_H */
