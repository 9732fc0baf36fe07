/*
 * zt_oracle.c -- CPU restatement of the reference's CPU twins for the fused
 * attention / RMSNorm path.  TEST INFRASTRUCTURE: the parity checker and the
 * CPU baseline.  The shipped library never links or calls this file.
 *
 * Followed, function by function (paths relative to the reference root):
 *   zto_attention_forward      src/attention.zig:60-153
 *   zto_attention_forward_at   src/cuda/attn_kernels.cu:233-283 (visibility),
 *                              src/attention.zig:111-149 (arithmetic)
 *   zto_attention_backward     src/autograd.zig:636-842
 *   zto_attention_backward_groups, zto_attention_forward_groups
 *                              the same two functions over whole kv groups,
 *                              parallel and bit-identical to the serial forms
 *   zto_attention_row_stats    src/autograd.zig:723-797 (the rebuild), with the
 *                              quantities src/cuda/attn_kernels.cu:520-532 keeps
 *   zto_attn_step              src/decode.zig:326-392
 *   zto_rmsnorm                src/norm.zig:14-47
 *   zto_rope                   src/rope.zig:21-55
 *   zto_rope_backward          src/autograd.zig:851-872
 *   zto_decode_step            src/decode.zig:244-270, src/kv_cache.zig:88-95
 *   zto_matmul                 src/tensor.zig:78-106
 *   zto_weight_grad            src/autograd.zig:958-972
 *   zto_input_grad             src/autograd.zig:999-1022
 * The generators are this build's own (splitmix64, Steele/Lea/Flood 2014, and
 * the Box-Muller transform); the reference used an LCG (src/cuda/attn_twin.zig:283-289).
 *
 * How each function is pinned is recorded in tests/test_oracle.py: the
 * reference's own known-answer tests (as fixtures in tests/golden/), closed
 * forms, brute force and finite differences.
 */
#include "zt_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int head_config_ok(int H, int Hkv, int D) {
    /* attention.zig:71-73 / autograd.zig:669-671 */
    return !(Hkv <= 0 || D <= 0 || H <= 0 || H % Hkv != 0);
}

/* One (batch, head) slab of attention.zig:111-149 for rows [t_begin, t_end). */
static void forward_head(const float *q, const float *k, const float *v, float *out, int T, int H,
                         int Hkv, int D, int h, int t_begin, int t_end, double *scores) {
    (void)T;
    const int group = H / Hkv;
    const int kv = h / group;
    const double scale = 1.0 / sqrt((double)D); /* attention.zig:87 */
    const size_t qc = (size_t)H * D, kc = (size_t)Hkv * D;
    for (int t = t_begin; t < t_end; ++t) {
        const float *q_head = q + (size_t)t * qc + (size_t)h * D;
        double row_max = -INFINITY;
        for (int s = 0; s <= t; ++s) { /* :117-124 */
            const float *k_head = k + (size_t)s * kc + (size_t)kv * D;
            double dot = 0;
            for (int j = 0; j < D; ++j) dot += (double)q_head[j] * (double)k_head[j];
            const double score = dot * scale;
            scores[s] = score;
            row_max = fmax(row_max, score);
        }
        double denom = 0; /* :128-133 */
        for (int s = 0; s <= t; ++s) {
            scores[s] = exp(scores[s] - row_max);
            denom += scores[s];
        }
        for (int s = 0; s <= t; ++s) scores[s] /= denom;
        float *out_row = out + (size_t)t * qc; /* :140-148 */
        for (int j = 0; j < D; ++j) {
            double acc = 0;
            for (int s = 0; s <= t; ++s) acc += scores[s] * (double)v[(size_t)s * kc + (size_t)kv * D + j];
            out_row[(size_t)h * D + j] = (float)acc;
        }
    }
}

int zto_attention_forward(const float *q, const float *k, const float *v, float *out, int B, int T,
                          int H, int Hkv, int D, int t_begin, int t_end) {
    return zto_attention_forward_mt(q, k, v, out, B, T, H, Hkv, D, t_begin, t_end, 1);
}

int zto_attention_forward_mt(const float *q, const float *k, const float *v, float *out, int B,
                             int T, int H, int Hkv, int D, int t_begin, int t_end, int n_threads) {
    if (!head_config_ok(H, Hkv, D)) return 1;
    if (T < 0 || B < 0 || t_begin < 0 || t_end > T || t_begin > t_end) return 2;
    const size_t qs = (size_t)T * H * D, ks = (size_t)T * Hkv * D;
    const int jobs = B * H;
#ifdef _OPENMP
    const int nt = n_threads > 0 ? n_threads : omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
#endif
    for (int job = 0; job < jobs; ++job) {
        const int b = job / H, h = job % H;
        double *scores = (double *)malloc(sizeof(double) * (size_t)(T > 0 ? T : 1));
        forward_head(q + b * qs, k + b * ks, v + b * ks, out + b * qs, T, H, Hkv, D, h, t_begin,
                     t_end, scores);
        free(scores);
    }
    (void)n_threads;
    return 0;
}

int zto_attention_forward_at(const float *q, const float *k, const float *v, float *out, int B,
                             int T, int H, int Hkv, int D, int q_offset, int n_keys) {
    if (!head_config_ok(H, Hkv, D)) return 1;
    if (T < 1 || q_offset < 0 || n_keys < 1 || q_offset > n_keys - T) return 2;
    const int group = H / Hkv;
    const double scale = 1.0 / sqrt((double)D);
    const size_t qc = (size_t)H * D, kc = (size_t)Hkv * D;
    double *scores = (double *)malloc(sizeof(double) * (size_t)n_keys);
    for (int b = 0; b < B; ++b) {
        const float *qb = q + (size_t)b * T * qc;
        const float *kb = k + (size_t)b * n_keys * kc;
        const float *vb = v + (size_t)b * n_keys * kc;
        float *ob = out + (size_t)b * T * qc;
        for (int h = 0; h < H; ++h) {
            const int kv = h / group;
            for (int t = 0; t < T; ++t) {
                const int last = q_offset + t; /* keys 0..last are visible */
                const float *q_head = qb + (size_t)t * qc + (size_t)h * D;
                double row_max = -INFINITY;
                for (int s = 0; s <= last; ++s) {
                    const float *k_head = kb + (size_t)s * kc + (size_t)kv * D;
                    double dot = 0;
                    for (int j = 0; j < D; ++j) dot += (double)q_head[j] * (double)k_head[j];
                    scores[s] = dot * scale;
                    row_max = fmax(row_max, scores[s]);
                }
                double denom = 0;
                for (int s = 0; s <= last; ++s) {
                    scores[s] = exp(scores[s] - row_max);
                    denom += scores[s];
                }
                for (int s = 0; s <= last; ++s) scores[s] /= denom;
                for (int j = 0; j < D; ++j) {
                    double acc = 0;
                    for (int s = 0; s <= last; ++s) acc += scores[s] * (double)vb[(size_t)s * kc + (size_t)kv * D + j];
                    ob[(size_t)t * qc + (size_t)h * D + j] = (float)acc;
                }
            }
        }
    }
    free(scores);
    return 0;
}

/* autograd.zig:735-820 for query row t of head h: the softmax rebuilt in f64
 * (probs[s], s <= t), d p and the Jacobian's dot, p_ds[s] = probs (dp - dot),
 * and dq[t] narrowed once.  Shared by the serial backward and the two-phase
 * group backward below, so both form every f64 value by the same operations. */
static void backward_row(const float *q, const float *k, const float *v, const float *dout, float *dq,
                         int H, int Hkv, int D, int h, int t, double *probs, double *d_probs, double *p_ds) {
    const int group = H / Hkv;
    const int kv = h / group;
    const double scale = 1.0 / sqrt((double)D); /* :691 */
    const size_t qc = (size_t)H * D, kc = (size_t)Hkv * D;
    const float *q_head = q + (size_t)t * qc + (size_t)h * D;
    const float *dh = dout + (size_t)t * qc + (size_t)h * D;
    /* Rebuild the softmax (:735-770).  The 8-way unroll there keeps every
     * value bit for bit what this scalar loop gives (:617-633). */
    double row_max = -INFINITY;
    for (int s = 0; s <= t; ++s) {
        const float *k_head = k + (size_t)s * kc + (size_t)kv * D;
        double dot = 0;
        for (int j = 0; j < D; ++j) dot += (double)q_head[j] * (double)k_head[j];
        probs[s] = dot * scale;
        row_max = fmax(row_max, probs[s]);
    }
    double denom = 0;
    for (int s = 0; s <= t; ++s) {
        probs[s] = exp(probs[s] - row_max);
        denom += probs[s];
    }
    for (int s = 0; s <= t; ++s) probs[s] /= denom;
    /* d p and the Jacobian's dot (:774-797). */
    double dot_pp = 0;
    for (int s = 0; s <= t; ++s) {
        const float *v_head = v + (size_t)s * kc + (size_t)kv * D;
        double acc = 0;
        for (int j = 0; j < D; ++j) acc += (double)dh[j] * (double)v_head[j];
        d_probs[s] = acc;
        dot_pp += probs[s] * acc;
    }
    for (int s = 0; s <= t; ++s) p_ds[s] = probs[s] * (d_probs[s] - dot_pp); /* :799 */
    /* d q[t]: f64 accumulate of (p_ds * k) * scale, one narrowing (:803-820). */
    for (int j = 0; j < D; ++j) {
        double acc = 0;
        for (int s = 0; s <= t; ++s) acc += p_ds[s] * (double)k[(size_t)s * kc + (size_t)kv * D + j] * scale;
        dq[(size_t)t * qc + (size_t)h * D + j] = (float)acc;
    }
}

/* autograd.zig:821-838: the f32 read-modify-write of one (t, s) term into
 * dk[s] and dv[s], from row t's p_ds[s] and probs[s]. */
static void backward_term(const float *q, const float *dout, float *dk, float *dv, int H, int Hkv, int D,
                          int h, int t, int s, double p_ds_s, double probs_s) {
    const int kv = h / (H / Hkv);
    const double scale = 1.0 / sqrt((double)D);
    const size_t qc = (size_t)H * D, kc = (size_t)Hkv * D;
    const float *q_head = q + (size_t)t * qc + (size_t)h * D;
    const float *dh = dout + (size_t)t * qc + (size_t)h * D;
    float *dk_row = dk + (size_t)s * kc + (size_t)kv * D;
    float *dv_row = dv + (size_t)s * kc + (size_t)kv * D;
    for (int j = 0; j < D; ++j) {
        dk_row[j] += (float)(p_ds_s * (double)q_head[j] * scale);
        dv_row[j] += (float)(probs_s * (double)dh[j]);
    }
}

/* autograd.zig:723-840 for one (batch, head), rows [t_begin, t_end). */
static void backward_head(const float *q, const float *k, const float *v, const float *dout,
                          float *dq, float *dk, float *dv, int T, int H, int Hkv, int D, int h,
                          int t_begin, int t_end, double *probs, double *d_probs, double *p_ds) {
    (void)T;
    for (int t = t_begin; t < t_end; ++t) {
        backward_row(q, k, v, dout, dq, H, Hkv, D, h, t, probs, d_probs, p_ds);
        for (int s = 0; s <= t; ++s) backward_term(q, dout, dk, dv, H, Hkv, D, h, t, s, p_ds[s], probs[s]);
    }
}

int zto_attention_backward(const float *q, const float *k, const float *v, const float *dout,
                           float *dq, float *dk, float *dv, int B, int T, int H, int Hkv, int D,
                           int t_begin, int t_end) {
    return zto_attention_backward_mt(q, k, v, dout, dq, dk, dv, B, T, H, Hkv, D, t_begin, t_end, 1);
}

int zto_attention_backward_mt(const float *q, const float *k, const float *v, const float *dout,
                              float *dq, float *dk, float *dv, int B, int T, int H, int Hkv, int D,
                              int t_begin, int t_end, int n_threads) {
    if (!head_config_ok(H, Hkv, D)) return 1;
    if (T < 0 || B < 0 || t_begin < 0 || t_end > T || t_begin > t_end) return 2;
    const size_t qs = (size_t)T * H * D, ks = (size_t)T * Hkv * D;
    memset(dk, 0, sizeof(float) * ks * (size_t)B);
    memset(dv, 0, sizeof(float) * ks * (size_t)B);
    const int group = H / Hkv;
    const int jobs = B * Hkv;
#ifdef _OPENMP
    const int nt = n_threads > 0 ? n_threads : omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
#endif
    for (int job = 0; job < jobs; ++job) {
        const int b = job / Hkv, kvh = job % Hkv;
        const size_t n = (size_t)(T > 0 ? T : 1);
        double *buf = (double *)malloc(sizeof(double) * 3 * n);
        /* The heads of one kv group in ascending order: the h -> t -> s order
         * of the reference's loop nest (:723-724), restricted to this group. */
        for (int h = kvh * group; h < (kvh + 1) * group; ++h)
            backward_head(q + b * qs, k + b * ks, v + b * ks, dout + b * qs, dq + b * qs, dk + b * ks,
                          dv + b * ks, T, H, Hkv, D, h, t_begin, t_end, buf, buf + n, buf + 2 * n);
        free(buf);
    }
    (void)n_threads;
    return 0;
}

/* The whole-group backward in two phases.  Phase 1 (parallel over rows):
 * backward_row for every (sequence, head of the groups, row t), keeping the
 * row's probs and p_ds in a packed lower triangle.  Phase 2 (parallel over
 * blocks of 8 key rows s): backward_term for every term that reaches those
 * rows, heads ascending, then t ascending -- for each dk/dv element the same
 * terms in the same order as the serial h -> t -> s loop nest (:723-838), so
 * every f32 rounding of the read-modify-write chain is the serial one. */
int zto_attention_backward_groups(const float *q, const float *k, const float *v, const float *dout,
                                  float *dq, float *dk, float *dv, int B, int T, int H, int Hkv, int D,
                                  int kv_begin, int kv_end, int n_threads) {
    if (!head_config_ok(H, Hkv, D)) return 1;
    if (T < 0 || B < 0 || kv_begin < 0 || kv_end > Hkv || kv_begin > kv_end) return 2;
    if (T == 0 || B == 0 || kv_begin == kv_end) return 0;
    const int group = H / Hkv;
    const int n_h = (kv_end - kv_begin) * group;  /* heads of the selected groups */
    const size_t qs = (size_t)T * H * D, ks = (size_t)T * Hkv * D, kc = (size_t)Hkv * D;
    const size_t tri = (size_t)T * (size_t)(T + 1) / 2;
    double *pp = (double *)malloc(sizeof(double) * tri * (size_t)n_h * (size_t)B);
    double *pd = (double *)malloc(sizeof(double) * tri * (size_t)n_h * (size_t)B);
    if (!pp || !pd) {
        free(pp);
        free(pd);
        return 3;
    }
    const size_t cols = sizeof(float) * (size_t)(kv_end - kv_begin) * D;  /* the groups' columns of a row */
    for (int b = 0; b < B; ++b) {
        for (int s = 0; s < T; ++s) {
            memset(dk + b * ks + (size_t)s * kc + (size_t)kv_begin * D, 0, cols);
            memset(dv + b * ks + (size_t)s * kc + (size_t)kv_begin * D, 0, cols);
        }
    }
#ifdef _OPENMP
    const int nt = n_threads > 0 ? n_threads : omp_get_max_threads();
#endif
    /* Phase 1: rows, heaviest (latest) first. */
    const long long rows = (long long)B * n_h * T;
#ifdef _OPENMP
#pragma omp parallel num_threads(nt)
#endif
    {
        double *d_probs = (double *)malloc(sizeof(double) * (size_t)T);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 4)
#endif
        for (long long job = 0; job < rows; ++job) {
            const int t = T - 1 - (int)(job % T);
            const int hi = (int)((job / T) % n_h), b = (int)(job / ((long long)T * n_h));
            const int h = kv_begin * group + hi;
            const size_t blk = ((size_t)b * n_h + hi) * tri + (size_t)t * (size_t)(t + 1) / 2;
            backward_row(q + b * qs, k + b * ks, v + b * ks, dout + b * qs, dq + b * qs, H, Hkv, D, h, t, pp + blk,
                         d_probs, pd + blk);
        }
        free(d_probs);
    }
    /* Phase 2: blocks of 8 key rows; within a block, per kv group, heads
     * ascending, t ascending, the block's rows s <= t. */
    const int n_sb = (T + 7) / 8;
    const long long jobs = (long long)B * n_sb;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
#endif
    for (long long job = 0; job < jobs; ++job) {
        const int b = (int)(job / n_sb), s0 = (int)(job % n_sb) * 8, s1 = s0 + 8 < T ? s0 + 8 : T;
        for (int kvh = kv_begin; kvh < kv_end; ++kvh)
            for (int h = kvh * group; h < (kvh + 1) * group; ++h) {
                const int hi = h - kv_begin * group;
                for (int t = s0; t < T; ++t) {
                    const size_t blk = ((size_t)b * n_h + hi) * tri + (size_t)t * (size_t)(t + 1) / 2;
                    const int s_hi = t + 1 < s1 ? t + 1 : s1;
                    for (int s = s0; s < s_hi; ++s)
                        backward_term(q + b * qs, dout + b * qs, dk + b * ks, dv + b * ks, H, Hkv, D, h, t, s,
                                      pd[blk + s], pp[blk + s]);
                }
            }
    }
    free(pp);
    free(pd);
    (void)n_threads;
    return 0;
}

/* All rows of the heads of kv groups [kv_begin, kv_end), parallel over
 * 16-row chunks: rows are independent (attention.zig:111-149), so this is
 * bit-identical to zto_attention_forward over those heads. */
int zto_attention_forward_groups(const float *q, const float *k, const float *v, float *out, int B, int T,
                                 int H, int Hkv, int D, int kv_begin, int kv_end, int n_threads) {
    if (!head_config_ok(H, Hkv, D)) return 1;
    if (T < 0 || B < 0 || kv_begin < 0 || kv_end > Hkv || kv_begin > kv_end) return 2;
    const int group = H / Hkv;
    const int n_h = (kv_end - kv_begin) * group, n_c = (T + 15) / 16;
    const size_t qs = (size_t)T * H * D, ks = (size_t)T * Hkv * D;
    const long long jobs = (long long)B * n_h * n_c;
#ifdef _OPENMP
    const int nt = n_threads > 0 ? n_threads : omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
#endif
    for (long long job = 0; job < jobs; ++job) {
        const int c = n_c - 1 - (int)(job % n_c);
        const int hi = (int)((job / n_c) % n_h), b = (int)(job / ((long long)n_c * n_h));
        double *scores = (double *)malloc(sizeof(double) * (size_t)T);
        const int t1 = 16 * c + 16 < T ? 16 * c + 16 : T;
        forward_head(q + b * qs, k + b * ks, v + b * ks, out + b * qs, T, H, Hkv, D, kv_begin * group + hi, 16 * c,
                     t1, scores);
        free(scores);
    }
    (void)n_threads;
    return 0;
}

int zto_attention_row_stats(const float *q, const float *k, const float *v, const float *dout,
                            double *row_max, double *row_den, double *row_del, int B, int T, int H,
                            int Hkv, int D) {
    if (!head_config_ok(H, Hkv, D)) return 1;
    const int group = H / Hkv;
    const double scale = 1.0 / sqrt((double)D);
    const size_t qc = (size_t)H * D, kc = (size_t)Hkv * D;
    double *sc = (double *)malloc(sizeof(double) * (size_t)(T > 0 ? T : 1));
    for (int b = 0; b < B; ++b)
        for (int h = 0; h < H; ++h) {
            const int kv = h / group;
            const float *qb = q + (size_t)b * T * qc, *db = dout + (size_t)b * T * qc;
            const float *kb = k + (size_t)b * T * kc, *vb = v + (size_t)b * T * kc;
            for (int t = 0; t < T; ++t) {
                double m = -INFINITY;
                for (int s = 0; s <= t; ++s) {
                    double dot = 0;
                    for (int j = 0; j < D; ++j)
                        dot += (double)qb[(size_t)t * qc + (size_t)h * D + j] * (double)kb[(size_t)s * kc + (size_t)kv * D + j];
                    sc[s] = dot * scale;
                    m = fmax(m, sc[s]);
                }
                double den = 0;
                for (int s = 0; s <= t; ++s) den += exp(sc[s] - m);
                double del = 0;
                for (int s = 0; s <= t; ++s) {
                    double dp = 0;
                    for (int j = 0; j < D; ++j)
                        dp += (double)db[(size_t)t * qc + (size_t)h * D + j] * (double)vb[(size_t)s * kc + (size_t)kv * D + j];
                    del += exp(sc[s] - m) / den * dp;
                }
                const size_t o = ((size_t)b * T + t) * H + h;
                row_max[o] = m;
                row_den[o] = den;
                row_del[o] = del;
            }
        }
    free(sc);
    return 0;
}

static void step_one(const float *q, const float *kc_, const float *vc_, float *out, int n_keys,
                      int H, int Hkv, int D, double *scores) {
    /* decode.zig:364-389 */
    const int group = H / Hkv;
    const double scale = 1.0 / sqrt((double)D);
    const size_t kc = (size_t)Hkv * D;
    for (int h = 0; h < H; ++h) {
        const int kv = h / group;
        const float *q_head = q + (size_t)h * D;
        double row_max = -INFINITY;
        for (int s = 0; s < n_keys; ++s) {
            const float *k_head = kc_ + (size_t)s * kc + (size_t)kv * D;
            double dot = 0;
            for (int j = 0; j < D; ++j) dot += (double)q_head[j] * (double)k_head[j];
            scores[s] = dot * scale;
            row_max = fmax(row_max, scores[s]);
        }
        double denom = 0;
        for (int s = 0; s < n_keys; ++s) {
            scores[s] = exp(scores[s] - row_max);
            denom += scores[s];
        }
        for (int s = 0; s < n_keys; ++s) scores[s] /= denom;
        for (int j = 0; j < D; ++j) {
            double a = 0;
            for (int s = 0; s < n_keys; ++s) a += scores[s] * (double)vc_[(size_t)s * kc + (size_t)kv * D + j];
            out[(size_t)h * D + j] = (float)a;
        }
    }
}

int zto_attn_step_mt(const float *q, const float *k_cache, const float *v_cache, float *out,
                     const int *n_keys, int B, int n_ctx, int H, int Hkv, int D, int n_threads) {
    if (!head_config_ok(H, Hkv, D)) return 1; /* decode.zig:339-341 */
    for (int b = 0; b < B; ++b)
        if (n_keys[b] < 1 || n_keys[b] > n_ctx) return 2; /* decode.zig:350 */
    const size_t cs = (size_t)n_ctx * Hkv * D, qs = (size_t)H * D;
#ifdef _OPENMP
    const int nt = n_threads > 0 ? n_threads : omp_get_max_threads();
#pragma omp parallel for schedule(dynamic, 1) num_threads(nt)
#endif
    for (int b = 0; b < B; ++b) {
        double *scores = (double *)malloc(sizeof(double) * (size_t)n_keys[b]);
        step_one(q + b * qs, k_cache + b * cs, v_cache + b * cs, out + b * qs, n_keys[b], H, Hkv, D, scores);
        free(scores);
    }
    (void)n_threads;
    return 0;
}

int zto_attn_step(const float *q, const float *k_cache, const float *v_cache, float *out,
                  const int *n_keys, int B, int n_ctx, int H, int Hkv, int D) {
    return zto_attn_step_mt(q, k_cache, v_cache, out, n_keys, B, n_ctx, H, Hkv, D, 1);
}

void zto_rmsnorm(const float *x, const float *w, float *y, int rows, int cols, double eps) {
    for (int r = 0; r < rows; ++r) {
        const float *x_row = x + (size_t)r * cols;
        float *y_row = y + (size_t)r * cols;
        double sum_sq = 0; /* norm.zig:28-29 */
        for (int i = 0; i < cols; ++i) sum_sq += (double)x_row[i] * (double)x_row[i];
        const float rms = (float)sqrt(sum_sq / (double)cols + eps); /* :41 */
        for (int i = 0; i < cols; ++i) y_row[i] = x_row[i] / rms * w[i]; /* :44, f32 */
    }
}

int zto_rope(const float *x, float *y, int rows, int cols, int pos, double theta, int head_dim) {
    if (head_dim <= 0 || head_dim % 2 != 0) return 1; /* rope.zig:28 */
    if (cols % head_dim != 0) return 2;                /* :29 */
    const int half = head_dim / 2;
    for (int r = 0; r < rows; ++r) {
        const float *src = x + (size_t)r * cols;
        float *dst = y + (size_t)r * cols;
        const double t = (double)(pos + r);
        for (int h = 0; h < cols / head_dim; ++h) {
            const int base = h * head_dim;
            for (int i = 0; i < half; ++i) {
                const double exponent = (double)(2 * i) / (double)head_dim; /* :43 */
                const double angle = t / pow(theta, exponent);
                const double c = cos(angle), s = sin(angle);
                const double lo = (double)src[base + i], hi = (double)src[base + i + half];
                dst[base + i] = (float)(lo * c - hi * s);
                dst[base + i + half] = (float)(hi * c + lo * s);
            }
        }
    }
    return 0;
}

int zto_rope_backward(const float *dout, float *din, int rows, int cols, int pos, double theta, int head_dim) {
    if (head_dim <= 0 || head_dim % 2 != 0) return 1;
    if (cols % head_dim != 0) return 2;
    const int half = head_dim / 2;
    for (int r = 0; r < rows; ++r) {
        const float *src = dout + (size_t)r * cols;
        float *dst = din + (size_t)r * cols;
        const double t = (double)(pos + r);
        for (int h = 0; h < cols / head_dim; ++h) {
            const int base = h * head_dim;
            for (int i = 0; i < half; ++i) {
                const double exponent = (double)(2 * i) / (double)head_dim; /* autograd.zig:861 */
                const double angle = t / pow(theta, exponent);
                const double c = cos(angle), s = sin(angle);
                const double lo = (double)src[base + i], hi = (double)src[base + i + half];
                dst[base + i] = (float)(lo * c + hi * s);        /* :867 */
                dst[base + i + half] = (float)(hi * c - lo * s); /* :868 */
            }
        }
    }
    return 0;
}

int zto_decode_step(const float *q, const float *k_new, const float *v_new, float *k_cache, float *v_cache,
                    float *out, const int *pos, int B, int n_ctx, int H, int Hkv, int D, double theta) {
    if (!head_config_ok(H, Hkv, D) || D % 2 != 0) return 1;
    for (int b = 0; b < B; ++b)
        if (pos[b] < 0 || pos[b] >= n_ctx) return 2; /* kv_cache.zig:91: Full */
    const size_t qs = (size_t)H * D, ks = (size_t)Hkv * D, cs = (size_t)n_ctx * ks;
    float *q_pos = (float *)malloc(sizeof(float) * qs);
    int rc = 0;
    for (int b = 0; b < B && rc == 0; ++b) {
        rc = zto_rope(q + b * qs, q_pos, 1, H * D, pos[b], theta, D);                                   /* decode.zig:244 */
        if (!rc) rc = zto_rope(k_new + b * ks, k_cache + b * cs + (size_t)pos[b] * ks, 1, Hkv * D, pos[b], theta, D);
        if (rc) break;
        memcpy(v_cache + b * cs + (size_t)pos[b] * ks, v_new + b * ks, sizeof(float) * ks);            /* :259 */
        const int nk = pos[b] + 1;
        rc = zto_attn_step(q_pos, k_cache + b * cs, v_cache + b * cs, out + b * qs, &nk, 1, n_ctx, H, Hkv, D);
    }
    free(q_pos);
    return rc;
}

/* out[i][j] = sum_k a[i][k] b[k][j]: one f32 accumulator per output element,
 * k ascending, each product rounded to f32 and then added (Zig's strict float
 * mode contracts nothing); the 8-lane unrolling of tensor.zig:84-93 does not
 * change any element's sequence. */
void zto_matmul(const float *a, const float *b, float *out, int M, int K, int N) {
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            float acc = 0.f;
            for (int k = 0; k < K; ++k) {
                const float prod = a[(size_t)i * K + k] * b[(size_t)k * N + j];
                acc += prod;
            }
            out[(size_t)i * N + j] = acc;
        }
}

/* w[i][j] += input[t][i] * dout[t][j], as an f32 read-modify-write per term,
 * i outer, t ascending, j inner (autograd.zig:960-969). */
void zto_weight_grad(float *w, const float *input, const float *dout, int T, int I, int J) {
    for (int i = 0; i < I; ++i)
        for (int t = 0; t < T; ++t) {
            const float scale = input[(size_t)t * I + i];
            for (int j = 0; j < J; ++j) {
                const float prod = scale * dout[(size_t)t * J + j];
                w[(size_t)i * J + j] += prod;
            }
        }
}

/* out[t][i] += sum_j dout[t][j] * w[i][j]: the sum in one f32 accumulator over
 * j ascending, added to out once (autograd.zig:1001-1020). */
void zto_input_grad(float *out, const float *dout, const float *w, int T, int J, int I) {
    for (int t = 0; t < T; ++t)
        for (int i = 0; i < I; ++i) {
            float acc = 0.f;
            for (int j = 0; j < J; ++j) {
                const float prod = dout[(size_t)t * J + j] * w[(size_t)i * J + j];
                acc += prod;
            }
            out[(size_t)t * I + i] += acc;
        }
}

uint64_t zto_splitmix64(uint64_t seed, uint64_t counter) {
    uint64_t z = seed + (counter + 1) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static double unit(uint64_t x) { return (double)(x >> 11) * 0x1.0p-53; }

void zto_fill_normal(float *out, size_t n, uint64_t seed, double mean, double sigma) {
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; ++i) {
        const double u1 = 1.0 - unit(zto_splitmix64(seed, 2 * (uint64_t)i)); /* (0, 1] */
        const double u2 = unit(zto_splitmix64(seed, 2 * (uint64_t)i + 1));
        const double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
        out[i] = (float)(mean + sigma * z);
    }
}

void zto_fill_uniform(float *out, size_t n, uint64_t seed, double lo, double hi) {
    for (size_t i = 0; i < n; ++i) out[i] = (float)(lo + (hi - lo) * unit(zto_splitmix64(seed, (uint64_t)i)));
}
