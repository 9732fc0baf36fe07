// Kernel argument blocks, shared by the device code (kernels/*.hip) and the
// host launcher (zt_attn.cpp), which passes each one as the single argument of
// hipModuleLaunchKernel.  Plain C layout: no HIP types.
#pragma once

struct FwdArgs {
    const float *q;    // [B, T, H*dim]
    const float *k;    // [B, kv_rows, Hkv*dim]
    const float *v;    // [B, kv_rows, Hkv*dim]
    float *out;        // [B, T, H*dim]
    float *lse;        // [B, T, H] log-sum-exp of each row's scaled scores, or null
    // If non-null (T = n_keys, q_offset 0), the scaled scores s = q k log2(e)/sqrt(dim)
    // of every 16 x 16 tile on or below the diagonal, unmasked, in the dS tile
    // order of BwdArgs::ds_out, for a dk/dv kernel that reads them back.
    float *s_out;
    int pair;          // a workgroup takes row tiles n_row_tiles - 1 - p and p
    int B, T, H, Hkv, dim;
    int q_offset, n_keys, kv_rows;
    int HW;            // query heads per workgroup (1, 2 or 4; divides H/Hkv)
    int n_row_tiles;   // ceil(T / (16 * 4 / HW))
    int n_head_blocks; // H / HW
    float scale_log2e; // log2(e) / sqrt(dim)
};

// Causal 16 x 16 score / dS tiles, packed by rows: row tile tb holds the tiles
// sb = 0..tb (none above the diagonal), tile (tb, sb) at tb (tb + 1) / 2 + sb of
// its (sequence, head) block of zt_tri_count(nt) tiles, nt = ceil(T / 16).
// constexpr: callable from the host launcher and from device code.
constexpr long long zt_tri_count(int nt) { return (long long)nt * (nt + 1) / 2; }
// Unsigned product: no sign fix-up for the halving (tb >= 0).
constexpr long long zt_tri_index(int tb, int sb) {
    return (long long)(((unsigned long long)(unsigned)tb * (unsigned)(tb + 1)) >> 1) + sb;
}

struct BwdArgs {
    const float *q, *k, *v, *dout;       // q/dout [B,T,H*dim]; k/v [B,T,Hkv*dim]
    float *dq, *dk, *dv;                 // assigned, never accumulated into
    float *row_max, *row_den, *row_del;  // [B,T,H]
    // Saved-statistics mode (lse non-null): the forward's output o and
    // log-sum-exp lse replace row_max / row_den; the dq kernel writes
    // row_del = sum_d o * dO itself.
    const float *o, *lse;
    // If non-null, the dk/dv kernel writes dS here in 16 x 16 tiles: tile
    // (b, h, t / 16, s / 16) at (b*H + h) * zt_tri_count(nt) + zt_tri_index(t/16, s/16)
    // (nt = ceil(T/16)), 256 floats in lane order (lane l, element r) =
    // (t = 16 tb + 4 (l >> 4) + r, s = 16 sb + (l & 15)); masked pairs are 0.
    // Tiles above the diagonal have no slot and are never written.
    // The score-reading dk/dv kernels (zt_bwd_dkdv8s_*, zt_bwd_dkdv_dmas_*)
    // find the forward's scaled scores (FwdArgs::s_out) in ds_out on entry;
    // each tile is read before its dS replaces it.
    float *ds_out;
    int B, T, H, Hkv, dim;
    int HW, n_row_tiles, n_head_blocks;  // dq kernel decomposition (as the forward)
    int HS, n_key_tiles;                 // dk/dv kernel: head split, ceil(T / (16 * 4/HS))
    int pair;                            // both kernels: a workgroup takes tiles p and n - 1 - p
    float scale, scale_log2e;
};

#define ZT_MAX_DIM 256  // the widest head the library admits
// Bytes of the fixed per-device scratch of zt_attn_decode_noalloc (noalloc.hip).
#define ZT_NOALLOC_SCRATCH_BYTES (16u << 20)
#define ZT_DEC_MAXB 64  // sequences per decode launch (n_keys travels in the arguments)

struct DecArgs {
    const float *q;   // [B, H*dim]
    const float *kc;  // [B, n_ctx, Hkv*dim]
    const float *vc;  // [B, n_ctx, Hkv*dim]
    float *out;       // [B, H*dim]
    float *part_acc;  // [B, H, n_chunks, dim]
    float *part_ml;   // [B, H, n_chunks, 2]
    int n_keys[ZT_DEC_MAXB];
    int b_base, nb, n_ctx, H, Hkv, dim;
    int chunk;     // keys per workgroup
    int n_chunks;  // chunk slots per (sequence, head) in the workspace
    int n_gsub;    // head sub-groups per kv group (group / G)
    float scale_log2e;
};

struct NormArgs {
    const float *x, *w;
    float *y;
    int rows, cols;
    double eps;
};

// RoPE over up to two row-aligned tensors sharing positions (q and k of one
// batch): tensor 1 has heads1 heads per row, tensor 2 heads2 (0 = absent).
// Row r sits at position pos + r % seq_len.
struct RopeArgs {
    const float *x1, *x2;
    float *y1, *y2;
    int rows, seq_len, heads1, heads2, pos, head_dim;
    double theta;
};

struct FillArgs {
    float *dst;
    unsigned long long n, seed;
    double p0, p1;  // normal: mean, sigma; uniform: lo, hi
};

// One decode step's cache update: RoPE on q and the new k at each sequence's
// position, the rotated k and the new v written into cache row pos[b].
struct AppendArgs {
    const float *q;      // [B, H*dim]   this step's query (before RoPE)
    const float *k;      // [B, Hkv*dim] this step's key (before RoPE)
    const float *v;      // [B, Hkv*dim]
    float *q_pos;        // [B, H*dim]   rotated query
    float *kc, *vc;      // [B, n_ctx, Hkv*dim] caches
    int pos[ZT_DEC_MAXB];
    int b_base, nb, n_ctx, H, Hkv, dim;
    double theta;
};

// Calibration probes (calibrate.hip).
struct CalArgs {
    const float *src;   // streaming-read source (16-byte aligned)
    unsigned long long n4;  // float4 elements to read
    float *out;         // one float per thread
    int iters;          // MFMA iterations per chain
};

// Dense f32 product C (+)= op(A) op(B) (gemm.hip).
struct GemmArgs {
    const float *a, *b;
    float *c;
    int M, N, K;
    int lda, ldb, ldc;     // row strides in floats of the matrices as stored
    int accumulate;        // 0: C = product; 1: C += product
    bool vec_a, vec_b;     // 16-byte loads allowed along the contiguous dimension
    bool vec_c;            // 16-byte stores allowed along C's rows
};

// dq from a stored dS (gemm.hip): dq[b, t, h, :] = scale * sum_{s <= t} dS[b, h, t, s] k[b, s, h / group, :].
struct DqDsArgs {
    const float *ds;   // dS in the tiled layout of BwdArgs::ds_out
    const float *k;    // [B, T, Hkv * dim]
    float *dq;         // [B, T, H * dim]
    int B, T, H, Hkv, dim;
    int tiles_m, tiles_n;  // row tiles; a workgroup takes tiles_m - 1 - p and p
    float scale;
    bool vec;          // 16-byte loads and stores along k and dq rows
};

