/*
 * zt_oracle.h -- CPU restatement of Z-TRANSFORMER's attention / RMSNorm / RoPE
 * CPU twins.  TEST INFRASTRUCTURE ONLY: this library is the parity checker and
 * the CPU baseline.  Nothing in the shipped library (z-transformer_amd/) links,
 * loads or calls it; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may.
 *
 * Every function restates one reference function; the file:line it follows is
 * given beside each declaration.  Arithmetic (f64 accumulators, f32 narrowing
 * points, loop order) follows the reference exactly.  Built with
 * -ffp-contract=off so no multiply-add is fused, as in Zig's strict float mode.
 *
 * All tensors are dense row-major f32 (src/tensor.zig:3-54).  The reference has
 * no batch dimension; B > 1 here is B independent sequences laid end to end.
 */
#ifndef ZT_ORACLE_H
#define ZT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/attention.zig:60-153 (forwardWith, null sink).  q/out [B,T,H*D],
 * k/v [B,T,Hkv*D].  Only query rows [t_begin, t_end) are computed (each row
 * sees its full causal prefix, so a row subset is exact for those rows); rows
 * outside are left untouched.  Returns 0, or 1 for InvalidHeadConfig
 * (attention.zig:71-73). */
int zto_attention_forward(const float *q, const float *k, const float *v, float *out, int B, int T,
                          int H, int Hkv, int D, int t_begin, int t_end);

/* Same, parallel over (batch, head) with OpenMP: every output element is
 * produced by the identical operation sequence, so results are bit-identical
 * to zto_attention_forward.  n_threads <= 0 uses the OpenMP default. */
int zto_attention_forward_mt(const float *q, const float *k, const float *v, float *out, int B,
                             int T, int H, int Hkv, int D, int t_begin, int t_end, int n_threads);

/* The forward at an offset, as src/cuda/attn_kernels.cu:233-283 defines it
 * (query row t sits at absolute position q_offset + t and sees keys
 * s <= q_offset + t, s < n_keys), with attention.zig's f64 arithmetic.
 * q/out [B,T,H*D], k/v [B,n_keys,Hkv*D]. */
int zto_attention_forward_at(const float *q, const float *k, const float *v, float *out, int B,
                             int T, int H, int Hkv, int D, int q_offset, int n_keys);

/* src/autograd.zig:636-842 (attentionBackward).  dq is f64-accumulated and
 * narrowed once (:803-820); dk/dv are f32 read-modify-write per term in
 * h -> t -> s order (:821-838).  Only query rows [t_begin, t_end) contribute:
 * dq rows in that range are exact, and with t_end == T, dk/dv rows
 * s >= t_begin are exact (a key row s receives terms only from t >= s).
 * dk/dv are zeroed here first (Tensor.init zeroes, :693-696); dq rows outside
 * the range are left untouched. */
int zto_attention_backward(const float *q, const float *k, const float *v, const float *dout,
                           float *dq, float *dk, float *dv, int B, int T, int H, int Hkv, int D,
                           int t_begin, int t_end);

/* Same, parallel over (batch, kv group).  A kv group's dk/dv are touched only
 * by its own query heads, so each element sees the same terms in the same
 * order: bit-identical to zto_attention_backward. */
int zto_attention_backward_mt(const float *q, const float *k, const float *v, const float *dout,
                              float *dq, float *dk, float *dv, int B, int T, int H, int Hkv, int D,
                              int t_begin, int t_end, int n_threads);

/* attentionBackward for every row of the heads of kv groups [kv_begin,
 * kv_end) (whole groups: a kv group's dk/dv receive terms only from its own
 * heads).  dq of those heads (all rows) and dk/dv of those groups (zeroed
 * first) are written; everything else is untouched.  Two phases, parallel:
 * the per-row softmax rebuild, then dk/dv in blocks of key rows with each
 * element's f32 read-modify-write chain in the serial h -> t -> s order, so
 * the result is bit-identical to zto_attention_backward (tested).  Holds
 * 16 * B * group * (kv_end - kv_begin) * T (T + 1) / 2 bytes while it runs.
 * Returns 3 if that memory cannot be had. */
int zto_attention_backward_groups(const float *q, const float *k, const float *v, const float *dout,
                                  float *dq, float *dk, float *dv, int B, int T, int H, int Hkv, int D,
                                  int kv_begin, int kv_end, int n_threads);

/* attention.forward for every row of the heads of kv groups [kv_begin, kv_end),
 * parallel over 16-row chunks; bit-identical to zto_attention_forward. */
int zto_attention_forward_groups(const float *q, const float *k, const float *v, float *out, int B, int T,
                                 int H, int Hkv, int D, int kv_begin, int kv_end, int n_threads);

/* Per-row softmax statistics the device backward keeps as scratch
 * (src/cuda/attn_kernels.cu:520-532): row_max = max_s score, row_den =
 * sum_s exp(score - row_max), row_del = sum_s p * dp, all in f64 from the
 * same rebuild attentionBackward does (autograd.zig:723-797).  [B,T,H]. */
int zto_attention_row_stats(const float *q, const float *k, const float *v, const float *dout,
                            double *row_max, double *row_den, double *row_del, int B, int T, int H,
                            int Hkv, int D);

/* src/decode.zig:326-392 (attnStep), batched: q/out [B,H*D]; caches
 * [B,n_ctx,Hkv*D]; sequence b attends its first n_keys[b] rows.  Returns 1 on
 * InvalidHeadConfig or an n_keys outside [1, n_ctx] (decode.zig:339-351). */
int zto_attn_step(const float *q, const float *k_cache, const float *v_cache, float *out,
                  const int *n_keys, int B, int n_ctx, int H, int Hkv, int D);
int zto_attn_step_mt(const float *q, const float *k_cache, const float *v_cache, float *out,
                     const int *n_keys, int B, int n_ctx, int H, int Hkv, int D, int n_threads);

/* src/norm.zig:18-47.  eps is src/norm.zig:14 (1e-5) unless the caller passes
 * another.  x/y [rows, cols], w [cols]. */
void zto_rmsnorm(const float *x, const float *w, float *y, int rows, int cols, double eps);

/* src/rope.zig:21-55.  x/y [rows, cols]; row r at position pos + r.
 * Returns 1 on OddHeadDim, 2 on DimensionMismatch. */
int zto_rope(const float *x, float *y, int rows, int cols, int pos, double theta, int head_dim);

/* src/autograd.zig:851-872 (ropeBackward): din = R^T dout, the transposed
 * half-split rotation at position pos + r.  Returns 1 / 2 as zto_rope. */
int zto_rope_backward(const float *dout, float *din, int rows, int cols, int pos, double theta, int head_dim);

/* One decode step per sequence, as src/decode.zig:244-270 orders it:
 * q_pos = rope(q, pos), k_pos = rope(k_new, pos) (src/rope.zig:21-55), the
 * cache append of (k_pos, v_new) at row pos (src/kv_cache.zig:88-95), then
 * attnStep over pos + 1 keys.  The caches are updated in place. */
int zto_decode_step(const float *q, const float *k_new, const float *v_new, float *k_cache, float *v_cache,
                    float *out, const int *pos, int B, int n_ctx, int H, int Hkv, int D, double theta);

/* src/tensor.zig:78-106 (matmul): out[M,N] = a[M,K] b[K,N], f32 accumulator,
 * k ascending, products rounded before the add. */
void zto_matmul(const float *a, const float *b, float *out, int M, int K, int N);
/* src/autograd.zig:958-972 (weightGrad): w[I,J] += input[T,I]^T dout[T,J], an
 * f32 read-modify-write per term, i -> t -> j. */
void zto_weight_grad(float *w, const float *input, const float *dout, int T, int I, int J);
/* src/autograd.zig:999-1022 (inputGrad): out[T,I] += dout[T,J] w[I,J]^T, one
 * f32 accumulator per element over j ascending, added once. */
void zto_input_grad(float *out, const float *dout, const float *w, int T, int J, int I);

/* Seeded inputs: splitmix64 counter stream -> Box-Muller.  Element i uses
 * the 64-bit outputs at counters 2i and 2i+1, so any element can be made on
 * its own.  out[i] = (float)(mean + sigma * z_i). */
void zto_fill_normal(float *out, size_t n, uint64_t seed, double mean, double sigma);
/* out[i] = (float)(lo + (hi - lo) * u_i), u_i in [0,1) from counter i. */
void zto_fill_uniform(float *out, size_t n, uint64_t seed, double lo, double hi);
uint64_t zto_splitmix64(uint64_t seed, uint64_t counter);

#ifdef __cplusplus
}
#endif
#endif
