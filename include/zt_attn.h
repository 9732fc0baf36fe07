/*
 * zt_attn.h -- C ABI of the MI355X (gfx950) fused causal GQA attention and
 * RMSNorm library, libzt_attn.so.
 *
 * The first six entry points keep the names, argument meaning, return values
 * and refusal order of the reference's C ABI in src/cuda/attn_kernels.cu
 * (mirrored by the Zig FFI in src/cuda/device.zig:58-105), so the reference's
 * device.Attn holder binds them unchanged once its three runtime externs
 * (cudaMalloc/Free/Memcpy, device.zig:112-117) are renamed to their hip*
 * twins.  The stream argument is a hipStream_t (NULL = the default stream).
 *
 * Conventions, as in the reference (attn_kernels.cu:18-54, 940-951):
 *   - device pointers in; the CALLER owns all memory; nothing here allocates;
 *   - return 0 = the launch was accepted (asynchronous: a device fault shows
 *     only at the caller's next synchronising call);
 *   - return 1 = refused, with the reason on stderr; never exit();
 *   - outputs (out, dq, dk, dv) are assigned, never accumulated into.
 * One difference, for non-finite inputs only.  The reference's loops never
 * read a masked key (src/attention.zig:117-147); here a masked pair's score is
 * replaced by -inf (so a non-finite K row never reaches an earlier query) but
 * its product with V is kept with weight 0, so an inf or NaN in V row s can
 * turn column d of up to 80 earlier rows (those sharing its staged key tile)
 * into NaN through 0 * inf, and in the backward their dq rows.  Rows before
 * that window, the other columns and the other KV heads are bit-identical to
 * a finite run; rows the reference reaches get what it gives; K/V rows at or
 * past n_keys are never read (a cache need not be cleared).
 * Layout: dense row-major f32 (src/tensor.zig:3-54): q/out/dout/dq are
 * [T, n_heads*dim], k/v/dk/dv are [T, n_kv_heads*dim]; query head h reads kv
 * head h / (n_heads / n_kv_heads) (src/attention.zig:111-112).
 *
 * Everything after the six is an extension with no reference counterpart and
 * says so.
 */
#ifndef ZT_ATTN_H
#define ZT_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same type as HIP's own hipStream_t (hip_runtime_api.h). */
typedef struct ihipStream_t *hipStream_t;

/* ---- The reference's six entry points -------------------------------- */

/* Replaces zt_attn_dim_ok, src/cuda/attn_kernels.cu:648-659.  1 iff dim is
 * even and in [32, 256]; prints nothing. */
int zt_attn_dim_ok(int dim);

/* Replace zt_attn_forward_shmem / zt_attn_bwd_dq_shmem /
 * zt_attn_bwd_dkdv_shmem, src/cuda/attn_kernels.cu:692-706.  Pure byte
 * counts: the LDS bytes per workgroup THIS library's kernel asks at head width
 * `dim` with its key tile capped at `tile` (a tile cap below 64 selects the
 * 32-key tile; `group_q` does not change this library's schedule and is
 * ignored here).  The dk/dv figure is the most that kernel asks at `dim`.
 * 0 for a width zt_attn_dim_ok refuses. */
size_t zt_attn_forward_shmem(int dim, int tile, int group_q);
size_t zt_attn_bwd_dq_shmem(int dim, int tile);
size_t zt_attn_bwd_dkdv_shmem(int dim);

/* Replaces zt_attn_forward, src/cuda/attn_kernels.cu:833-938.
 * out[t] for query rows t in [0, T) at absolute positions q_offset + t, over
 * keys s <= q_offset + t, s < n_keys (k/v hold at least n_keys rows).  One
 * query row (T = 1, the reference's decode route, src/decode.zig:462) runs the
 * decode kernel over the q_offset + 1 visible keys, one chunk per workgroup,
 * with no workspace.
 * Refusal order: T < 1; width; group; n_heads > 65535; group_q outside
 * [1, 64] or dim*group_q > 1024; q_offset < 0 || n_keys < 1 ||
 * q_offset > n_keys - T; max_tile < 1; device LDS ceiling unreadable; no
 * tile fits.  group_q is validated exactly as the reference does and
 * otherwise has no effect (every wave owns 16 query rows). */
int zt_attn_forward(const float *q, const float *k, const float *v, float *out, int T, int n_heads,
                    int n_kv_heads, int dim, int group_q, int max_tile, int q_offset, int n_keys,
                    hipStream_t stream);

/* Replaces zt_attn_backward, src/cuda/attn_kernels.cu:952-1036.
 * dq [T, n_heads*dim], dk/dv [T, n_kv_heads*dim]; row_max/row_den/row_del are
 * [T, n_heads] scratch that the first kernel writes (max score, softmax
 * denominator exp-sum, and delta = sum_s p*dp) and the second reads on the
 * same stream.  Refusal order: T < 1; width; group; n_heads > 65535;
 * max_tile < 1; LDS ceiling unreadable; no tile fits. */
int zt_attn_backward(const float *q, const float *k, const float *v, const float *dout, float *dq,
                     float *dk, float *dv, float *row_max, float *row_den, float *row_del, int T,
                     int n_heads, int n_kv_heads, int dim, int max_tile, hipStream_t stream);

/* ---- Extensions (no reference counterpart) ---------------------------- */

/* Batched forward: B independent sequences.  q/out [B, T, n_heads*dim];
 * k/v [B, kv_rows, n_kv_heads*dim] (kv_rows >= n_keys rows per sequence, so a
 * preallocated cache can be passed whole).  Same semantics and refusals as
 * zt_attn_forward per sequence, plus B < 1 and kv_rows < n_keys. */
int zt_attn_forward_batched(const float *q, const float *k, const float *v, float *out, int B, int T,
                            int n_heads, int n_kv_heads, int dim, int group_q, int max_tile,
                            int q_offset, int n_keys, int kv_rows, hipStream_t stream);

/* Batched backward: q/dout/dq [B, T, n_heads*dim]; k/v/dk/dv
 * [B, T, n_kv_heads*dim]; row_* [B, T, n_heads]. */
int zt_attn_backward_batched(const float *q, const float *k, const float *v, const float *dout,
                             float *dq, float *dk, float *dv, float *row_max, float *row_den,
                             float *row_del, int B, int T, int n_heads, int n_kv_heads, int dim,
                             int max_tile, hipStream_t stream);

/* The two stages of zt_attn_backward_batched, for callers that schedule them
 * apart (and for per-stage timing).  zt_attn_bwd_dq writes dq and the row
 * statistics; zt_attn_bwd_dkdv reads those statistics and writes dk/dv, so on
 * one stream dq must run first.  Same layouts and refusals as the batched
 * backward (dkdv uses the default tile cap). */
int zt_attn_bwd_dq(const float *q, const float *k, const float *v, const float *dout, float *dq, float *row_max,
                   float *row_den, float *row_del, int B, int T, int n_heads, int n_kv_heads, int dim, int max_tile,
                   hipStream_t stream);
int zt_attn_bwd_dkdv(const float *q, const float *k, const float *v, const float *dout, float *dk, float *dv,
                     const float *row_max, const float *row_den, const float *row_del, int B, int T, int n_heads,
                     int n_kv_heads, int dim, hipStream_t stream);

/* Decode step over a KV cache, split over the key axis.  q/out [B, n_heads*dim];
 * k_cache/v_cache [B, n_ctx, n_kv_heads*dim] (the src/kv_cache.zig:58-63
 * layout per sequence); sequence b attends its first n_keys[b] cached rows,
 * its query sitting at position n_keys[b]-1 (src/decode.zig:326-392).
 * n_keys is a HOST array of B ints in [1, n_ctx].  `workspace` is device
 * memory of at least zt_attn_decode_workspace(...) bytes (chunk partials),
 * 16-byte aligned (as every workspace here; hipMalloc's are).
 * Refuses B < 1, n_ctx < 1, a refused width or group, an n_keys outside
 * [1, n_ctx], a null pointer, or a short workspace. */
size_t zt_attn_decode_workspace(int B, int n_ctx, int n_heads, int n_kv_heads, int dim);
int zt_attn_decode(const float *q, const float *k_cache, const float *v_cache, float *out,
                   const int *n_keys, int B, int n_ctx, int n_heads, int n_kv_heads, int dim,
                   void *workspace, size_t workspace_bytes, hipStream_t stream);

/* zt_attn_decode without a workspace.  No reference counterpart: it is for
 * callers that cannot allocate (code under graph capture, tight serving loops,
 * harnesses that forbid allocation).  The chunk partials go to a scratch array
 * of ZT_NOALLOC_SCRATCH_BYTES = 16 MiB that is part of the library's device
 * image, one copy per GPU, held until the process ends; the call allocates
 * nothing (no hipMalloc, no allocating library routine).  Same arguments,
 * semantics and refusals as zt_attn_decode, plus a refusal when the split's
 * partials exceed the scratch (every shape at the default split fits; only a
 * wider split forced with ZT_DEC_WGS can exceed it).  No part of the scratch
 * needs to start at zero: the combine reads only partials the same call wrote.
 * Every call on one GPU shares that GPU's scratch, so calls that overlap on
 * one GPU (concurrent streams, threads) race: serialise them.
 * Set-up: the library's first call of any entry point on a device loads its
 * code objects there (hipModuleLoadData), looks up the scratch's address and
 * resolves the decode kernels; that first call is not allocation-free.  Make
 * one call on each device outside graph capture (any entry point, e.g. a
 * warm-up zt_attn_decode_noalloc); every later call only launches. */
int zt_attn_decode_noalloc(const float *q, const float *k_cache, const float *v_cache, float *out,
                           const int *n_keys, int B, int n_ctx, int n_heads, int n_kv_heads, int dim,
                           hipStream_t stream);

/* One decode step with the KV cache resident on the device (no counterpart:
 * the reference re-uploads the whole prefix every step, src/decode.zig:435-437).
 * For each sequence b: RoPE (src/rope.zig:21-55, theta e.g. 500000) rotates
 * q[b] and k_new[b] at position pos[b]; the rotated key and v_new[b] are
 * written into cache row pos[b] (the src/kv_cache.zig:88-131 append: the cache
 * stores post-RoPE keys); then out[b] attends the first pos[b] + 1 rows, as
 * src/decode.zig:206-298 does per layer.  q/out [B, n_heads*dim], k_new/v_new
 * [B, n_kv_heads*dim], caches [B, n_ctx, n_kv_heads*dim]; pos is a HOST array
 * of B ints in [0, n_ctx) (a full cache is refused, kv_cache.zig:91).
 * `workspace` holds zt_attn_decode_step_workspace(...) bytes, 16-byte aligned. */
size_t zt_attn_decode_step_workspace(int B, int n_ctx, int n_heads, int n_kv_heads, int dim);
int zt_attn_decode_step(const float *q, const float *k_new, const float *v_new, float *k_cache, float *v_cache,
                        float *out, const int *pos, int B, int n_ctx, int n_heads, int n_kv_heads, int dim,
                        double theta, void *workspace, size_t workspace_bytes, hipStream_t stream);

/* RMSNorm, src/norm.zig:18-47 on the device (the reference's src/cuda/norm.cu
 * kernel has no C entry point).  x/y [rows, cols], w [cols]; eps is
 * src/norm.zig:14's 1e-5 for the reference's behaviour.  rows == 0 launches
 * nothing and returns 0 (norm.forward on zero rows is an empty result);
 * refuses rows < 0, cols < 1, eps < 0, null pointers. */
int zt_rmsnorm_forward(const float *x, const float *w, float *y, int rows, int cols, double eps,
                       hipStream_t stream);

/* RoPE, src/rope.zig:21-55 on the device (input preparation: Q/K rotated
 * before attention).  x/y [rows, cols], row r at position pos + r.  Refuses
 * an odd or non-positive head_dim (rope.zig:28) and cols % head_dim != 0
 * (rope.zig:29). */
int zt_rope_forward(const float *x, float *y, int rows, int cols, int pos, double theta,
                    int head_dim, hipStream_t stream);

/* ---- Training path with saved statistics (no reference counterpart) ----
 * The reference backward (zt_attn_backward above) rebuilds every row's softmax
 * statistics itself, which costs its dq kernel a fourth matmul.  A training
 * step that has just run the forward can keep them instead:
 *   zt_attn_forward_train  = zt_attn_forward (causal, q_offset 0, n_keys T,
 *       B sequences) that also writes lse[B, T, n_heads], each row's natural
 *       log-sum-exp of its scaled scores;
 *   zt_attn_backward_train = the same dq/dk/dv as zt_attn_backward from
 *       (q, k, v, out, dout, lse); delta [B, T, n_heads] is caller scratch
 *       (receives sum_d out * dout per row).  dq/dk/dv are assigned.
 * Same refusals as the reference entry points; the two stages are also
 * callable on their own (dq + delta first, then dk/dv on the same stream). */
int zt_attn_forward_train(const float *q, const float *k, const float *v, float *out, float *lse, int B, int T,
                          int n_heads, int n_kv_heads, int dim, hipStream_t stream);
int zt_attn_backward_train(const float *q, const float *k, const float *v, const float *out, const float *dout,
                           const float *lse, float *dq, float *dk, float *dv, float *delta, int B, int T,
                           int n_heads, int n_kv_heads, int dim, hipStream_t stream);
int zt_attn_bwd_dq_train(const float *q, const float *k, const float *v, const float *out, const float *dout,
                         const float *lse, float *dq, float *delta, int B, int T, int n_heads, int n_kv_heads,
                         int dim, hipStream_t stream);
int zt_attn_bwd_dkdv_train(const float *q, const float *k, const float *v, const float *out, const float *dout,
                           const float *lse, const float *delta, float *dk, float *dv, int B, int T, int n_heads,
                           int n_kv_heads, int dim, hipStream_t stream);
/* The same backward with dq formed from a stored dS instead of a third
 * kernel that rebuilds it: the dk/dv kernel writes dS[b, h, t, s] for every
 * causal pair into the workspace, and dq = dS k / sqrt(d) is then one causal
 * product per head.  Deterministic like the rest.  workspace: 16-byte aligned,
 * at least zt_attn_backward_train_workspace(...) bytes: delta, then the
 * causal 16 x 16 tiles of dS only, B * H * nt (nt + 1) / 2 of them with
 * nt = ceil(T / 16) (1.0 GiB at T = 4096 with 32 heads; 4.0 GiB at T = 8192).
 * stage: 1 = delta + dk/dv (+ dS), 2 = dq from dS, 3 = both; | ZT_WS_SCORES
 * when the workspace holds the scores zt_attn_forward_train_ws wrote for these
 * q, k (the dk/dv kernel then reads each score tile and overwrites it with dS
 * instead of forming Q K^T again).  ZT_WS_SCORES is single use: it is for
 * the first stage 1 after the zt_attn_forward_train_ws of the same q, k (the
 * same pointers) and shape on the same device; after that stage 1 the tiles
 * hold dS.  The library keeps a host-side record of which workspace holds
 * whose scores (set by zt_attn_forward_train_ws, consumed by the stage 1 that
 * reads them, dropped by a stage 1 that overwrites them) and refuses with 1
 * a ZT_WS_SCORES stage 1 that does not match it, rather than reading stale
 * tiles.  It cannot see q or k rewritten in place between the two calls;
 * that leaves out and lse stale as well.  No reference counterpart. */
#define ZT_WS_SCORES 4
size_t zt_attn_backward_train_workspace(int B, int T, int n_heads, int n_kv_heads, int dim);
int zt_attn_backward_train_ws(const float *q, const float *k, const float *v, const float *out, const float *dout,
                              const float *lse, float *dq, float *dk, float *dv, void *workspace,
                              size_t workspace_bytes, int B, int T, int n_heads, int n_kv_heads, int dim, int stage,
                              hipStream_t stream);
/* zt_attn_forward_train that also leaves the scaled scores q k log2(e)/sqrt(d)
 * of every causal 16 x 16 tile in the workspace's dS tiles, for
 * zt_attn_backward_train_ws(..., stage | ZT_WS_SCORES, ...).  Scores are kept
 * for the shapes whose dk/dv kernel reads them: an even number of query heads
 * per kv head with head_dim % 4 == 0 and head_dim <= 128 or a multiple of 32;
 * and head groups that cannot be halved (MHA, odd groups) with head_dim 32,
 * 64, 96 or 128 where the grid gives at most one paired dk/dv workgroup per
 * CU (the row-split kernel's shapes).  For the others this is
 * zt_attn_forward_train and ZT_WS_SCORES is ignored (so it is for q or dout
 * rows that are not 16-byte aligned).  The workspace is the
 * backward's (zt_attn_backward_train_workspace bytes).  No reference
 * counterpart. */
int zt_attn_forward_train_ws(const float *q, const float *k, const float *v, float *out, float *lse, void *workspace,
                             size_t workspace_bytes, int B, int T, int n_heads, int n_kv_heads, int dim,
                             hipStream_t stream);
/* Kernel names the training path (zt_attn_forward_train_ws +
 * zt_attn_backward_train_ws with ZT_WS_SCORES) launches for a shape, as
 * zt_attn_plan. */
int zt_attn_plan_train(int B, int T, int n_heads, int n_kv_heads, int dim, char *fwd, char *dq, char *dkdv,
                       size_t len);

/* RoPE backward, src/autograd.zig:851-872 on the device: din = R^T dout at
 * position pos + r (the gradient through zt_rope_forward), so an attention
 * block's backward -- zt_attn_backward then this on dq and dk -- stays on the
 * device.  Same layout and refusals as zt_rope_forward. */
int zt_rope_backward(const float *dout, float *din, int rows, int cols, int pos, double theta, int head_dim,
                     hipStream_t stream);

/* RoPE of q and k in one launch, as the model rotates both before attention
 * (src/model.zig:372-377; each is src/rope.zig:21-55): q/q_out [B, T, n_heads*head_dim],
 * k/k_out [B, T, n_kv_heads*head_dim], row t of every sequence at position pos + t.
 * One f64 angle per (position, pair) serves every head of both tensors.
 * In-place (q_out == q, k_out == k) is allowed.  No reference counterpart. */
int zt_rope_qk_forward(const float *q, const float *k, float *q_out, float *k_out, int B, int T, int n_heads,
                       int n_kv_heads, int head_dim, int pos, double theta, hipStream_t stream);

/* The transpose, for dq and dk together (src/autograd.zig:566-569 applies
 * ropeBackward to each).  No reference counterpart. */
int zt_rope_qk_backward(const float *dq, const float *dk, float *dq_out, float *dk_out, int B, int T,
                        int n_heads, int n_kv_heads, int head_dim, int pos, double theta, hipStream_t stream);

/* ---- Dense products of the model step (no reference C entry point) ----
 * src/tensor.zig:78-106 (tensor.matmul) on the device: out[M,N] = a[M,K] b[K,N],
 * row-major f32, FP32 MFMA with f32 accumulation (the reference reduces in f32
 * too, src/tensor_test.zig:185-273; only the rounding order differs).  K = 0
 * writes zeros; M = 0 or N = 0 writes nothing.  The reference's
 * DimensionMismatch is the caller's shape check (sizes are explicit here). */
int zt_matmul(const float *a, const float *b, float *out, int M, int K, int N, hipStream_t stream);
/* src/autograd.zig:958-972 (weightGrad): w[I,J] += input[T,I]^T dout[T,J]. */
int zt_weight_grad(float *w, const float *input, const float *dout, int T, int I, int J, hipStream_t stream);
/* src/autograd.zig:999-1022 (inputGrad): din[T,I] += dout[T,J] w[I,J]^T. */
int zt_input_grad(float *din, const float *dout, const float *w, int T, int J, int I, hipStream_t stream);
/* The kernel zt_matmul launches for an M x K x N product on the current device
 * ("zt_gemm_nn_<tile>" slab kernel or "zt_gemm_nn_sk<tile>" split-K kernel;
 * the two gradients take the same choice for the same output shape and
 * reduction length), into name[len].  0, or 1 if there is no usable device,
 * the shape is empty or name is too short.  No reference counterpart. */
int zt_matmul_plan(int M, int K, int N, char *name, int len);

/* Roofline calibration (no reference counterpart): the FP32 MFMA rate this
 * device sustains (two interleaved v_mfma_f32_16x16x4_f32 chains per wave,
 * four waves per SIMD) and the HBM rate of a streaming 16-byte-load read of
 * `src` (the decode kernel's access pattern), each the minimum time of three
 * runs after a warm-up.  scratch: one float per probe thread (>= 2048 * 256 * 4
 * bytes).  Synchronises the stream. */
int zt_calibrate(const float *src, size_t src_bytes, float *scratch, size_t scratch_bytes, double *mfma_tflops,
                 double *read_gbs, hipStream_t stream);

/* Launch floor (no reference counterpart): `launches` back-to-back launches of
 * an empty kernel of `blocks` workgroups x `threads` on `stream`, the average
 * microseconds per launch (minimum of three timings after a warm-up): what a
 * latency-bound kernel of that grid cannot go below.  Synchronises the stream. */
int zt_calibrate_launch(unsigned blocks, unsigned threads, int launches, double *us_per_launch, hipStream_t stream);

/* Seeded synthetic inputs (splitmix64 counter stream + Box-Muller): element i
 * depends only on (seed, i).  normal: mean + sigma*z; uniform: [lo, hi). */
int zt_fill_normal(float *dst, size_t n, uint64_t seed, double mean, double sigma, hipStream_t stream);
int zt_fill_uniform(float *dst, size_t n, uint64_t seed, double lo, double hi, hipStream_t stream);

/* The kernel names this library launches for a forward and a backward at
 * this shape on the current device (for profilers and benchmarks), each
 * written NUL-terminated into a buffer of `len` bytes.  1 if the shape is
 * refused or no device is usable. */
int zt_attn_plan(int B, int T, int n_heads, int n_kv_heads, int dim, int max_tile, char *fwd, char *dq,
                 char *dkdv, size_t len);

/* Tuning variables (no reference counterpart; process-wide).  Every kernel
 * variant is chosen from the shape; a sweep or a test may force one with
 * zt_attn_set_tuning(name, value), and value -1 returns the variable to the
 * shape rule.  Names and admitted values:
 *   ZT_ATTN_BK 32|64 (keys per staged K/V tile: forward, dq kernels),
 *   ZT_ATTN_FWD_W 4|8 (forward waves), ZT_ATTN_FPF 0|1 (forward register
 *   prefetch), ZT_ATTN_FPAIR 0|1 (paired forward row tiles), ZT_ATTN_QPF 0|1
 *   and ZT_ATTN_DQ_W 4|8 (dq kernel prefetch and waves), ZT_ATTN_HS 1|2|4
 *   (dk/dv head split), ZT_ATTN_W8 0|1 and ZT_ATTN_PF 0|1 (eight-wave dk/dv,
 *   its prefetch), ZT_ATTN_DMA 0|1 (asynchronously staged dk/dv),
 *   ZT_ATTN_BPAIR 0|1 (paired dq / dk/dv tiles), ZT_ATTN_DSPLIT 0|1
 *   (column-split dk/dv), ZT_ATTN_RSPLIT 0|1 (row-split dk/dv), ZT_DEC_WGS
 *   256..32768 (decode workgroup target), ZT_GEMM_TILE 32|64|128 (dense
 *   product slab tile), ZT_GEMM_SK 0|4|8|16 (dense product split-K waves, 0 =
 *   the slab kernels), ZT_GEMM_SK_TILE 16|32 (split-K tile), ZT_DQDS_TILE
 *   64|128 (dq-from-dS product tile), ZT_ROW_G
 *   1|2|4|8 and ZT_ROW_W 4|8 (query heads and waves per workgroup of the
 *   one-row forward, T = 1), ZT_ATTN_FKS 1|2 (key parts of the forward for
 *   one query head per workgroup: 2 = the key-split eight-wave kernel),
 *   ZT_DQDS_K 1|2 (key parts of the dq-from-dS product), ZT_ATTN_RSCORES
 *   0|1 (the row-split dk/dv kernel reading the forward's scores for head
 *   groups that cannot be halved; 0 = it forms S again and the forward keeps
 *   none).
 * Returns 0, or 1 (reason on stderr) for an unknown name or value.  The
 * process environment is never read.  Not synchronised with launches in
 * flight on other threads: set before launching. */
int zt_attn_set_tuning(const char *name, int value);
/* The forced value of a tuning variable, -1 when it follows the shape rule,
 * -2 for an unknown name. */
int zt_attn_get_tuning(const char *name);

/* Library version string, and the LDS ceiling per workgroup the library read
 * for the current device (0 = no usable device / code object). */
const char *zt_attn_version(void);
size_t zt_attn_lds_limit(void);

#ifdef __cplusplus
}
#endif
#endif
