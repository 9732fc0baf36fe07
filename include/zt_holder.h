/*
 * zt_holder.h -- the host-side holder of the reference's Zig FFI
 * (src/cuda/device.zig:119-501), restated in C++ over the zt_attn C ABI, plus
 * a C face of it so foreign callers (and this repository's tests) can drive it.
 *
 * The holder owns the eleven device buffers a forward/backward pass at one
 * shape needs (device.zig:185-212), sizes them once with overflow-checked
 * arithmetic, validates every call before it reaches the device, and maps each
 * failure to one of the reference's five errors (device.zig:119-141).
 * Allocation goes through hipMalloc/hipFree/hipMemcpy, the HIP twins of the
 * three runtime externs the reference binds (device.zig:112-117).
 */
#ifndef ZT_HOLDER_H
#define ZT_HOLDER_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* device.zig:119-141.  0 is success. */
enum zt_error {
    ZT_OK = 0,
    ZT_DEGENERATE_SHAPE = 1,
    ZT_SHAPE_TOO_LARGE = 2,
    ZT_CONFIG_REFUSED = 3,
    ZT_DEVICE_ALLOC_FAILED = 4,
    ZT_DEVICE_TRANSFER_FAILED = 5,
};

/* device.zig:143-160 (Kind). */
enum zt_kind { ZT_QUERY_HEADED = 0, ZT_KV_HEADED = 1, ZT_PER_ROW = 2 };

/* device.zig:162-171 (bytesFor): bytes of one buffer of `kind`. */
int zt_bytes_for(int kind, size_t t, size_t n_heads, size_t n_kv_heads, size_t dim, size_t *out);
/* device.zig:179-182 (toCInt). */
int zt_to_cint(size_t x, int *out);
/* device.zig:489-501 (forwardBounds): ZT_OK or ZT_SHAPE_TOO_LARGE. */
int zt_forward_bounds(int c_t, int q_offset, int n_keys, int t);

/* The buffers of a holder, in device.zig's field order (:186-196). */
enum zt_buffer {
    ZT_BUF_Q = 0, ZT_BUF_K, ZT_BUF_V, ZT_BUF_OUT, ZT_BUF_DOUT, ZT_BUF_DQ, ZT_BUF_DK, ZT_BUF_DV,
    ZT_BUF_ROW_MAX, ZT_BUF_ROW_DEN, ZT_BUF_ROW_DEL, ZT_N_BUFFERS
};

typedef struct zt_holder zt_holder;

/* device.zig:221-299 (Attn.init): refuses via zt_attn_dim_ok and the group
 * check BEFORE allocating; on an allocation failure frees what it took.
 * Beyond the eleven buffers the holder takes two workspaces, neither of
 * which is needed for correctness (a failed allocation is no error):
 *   - here, the one-row forward's chunk partials (zt_attn_decode_workspace
 *     bytes for one sequence of t rows: 1.0 MiB at t = 8192 with 32 heads,
 *     d = 128); without them see zt_holder_forward_at;
 *   - at the first whole-shape forward (zt_holder_forward), the score
 *     workspace of the saved-statistics backward
 *     (zt_attn_backward_train_workspace bytes for one sequence of t rows:
 *     1.0 GiB at t = 4096 with 32 heads, 4.0 GiB at 8192), only when it is at
 *     most a quarter of the device's free memory (hipMemGetInfo) then; a
 *     holder that only decodes never takes it; without it see
 *     zt_holder_backward.
 * zt_holder_workspace_bytes reports what is taken, beside
 * zt_holder_total_bytes's eleven buffers: budget VRAM with the sum. */
int zt_holder_init(size_t t, size_t n_heads, size_t n_kv_heads, size_t dim, zt_holder **out);
/* The same holder running the reference entry points only (zt_attn_forward,
 * also for one query row, then zt_attn_backward, which rebuilds the
 * statistics): no workspace at all, and
 * row_max / row_den hold the reference's max and denominator.  No reference
 * counterpart (device.zig has one mode). */
int zt_holder_init_exact(size_t t, size_t n_heads, size_t n_kv_heads, size_t dim, zt_holder **out);
void zt_holder_deinit(zt_holder *h);                                   /* :328-330 */
/* :332-341: the eleven buffers' bytes, as the reference counts them (the
 * workspaces are not included: zt_holder_workspace_bytes). */
size_t zt_holder_total_bytes(const zt_holder *h);
/* Bytes of the optional workspaces the holder holds now (0 for
 * zt_holder_init_exact).  No reference counterpart. */
size_t zt_holder_workspace_bytes(const zt_holder *h);
/* A buffer's writable device pointer.  Asking for q, k, v, out or row_max
 * drops the forward's saved state, as an upload does (the caller may now
 * change what the forward saw), so the next backward rebuilds the statistics;
 * the other buffers leave it.  To read without that, use zt_holder_buffer_ro. */
float *zt_holder_buffer(const zt_holder *h, int which);
/* The same pointer, read-only: keeps the saved state.  No reference
 * counterpart. */
const float *zt_holder_buffer_ro(const zt_holder *h, int which);
/* :376-379.  The whole-cache forward.  It also keeps what the backward would
 * otherwise rebuild (device.zig:400-402 requires the forward to run first on
 * the same buffers): row_max receives each row's log-sum-exp and row_den 1.0,
 * so p = exp(score - row_max) / row_den as in the reference's scratch, and the
 * scores go to the holder's workspace.  group_q and max_tile are admitted as
 * zt_attn_forward admits them (an argument it refuses is refused the same way). */
int zt_holder_forward(const zt_holder *h, int group_q, int max_tile);
/* :381-398.  forward_at with q_offset 0, n_keys t_cap and t t_cap is
 * zt_holder_forward; any other (decode-shaped) call drops the saved state and
 * runs zt_attn_forward, except one query row (t = 1, the reference's decode
 * seam, src/decode.zig:462) on a holder from zt_holder_init with its chunk
 * partials: that runs zt_attn_decode over the q_offset + 1 visible cache rows,
 * keys split into chunks across the device (the one-row zt_attn_forward gives
 * a single sequence only one workgroup per kv head and head sub-group).  Same
 * result to rounding; group_q and max_tile are admitted as zt_attn_forward
 * admits them. */
int zt_holder_forward_at(const zt_holder *h, int group_q, int max_tile, int q_offset, int n_keys,
                         int t);
/* :400-406.  dq, dk, dv from the buffers.  After zt_holder_forward with no
 * upload into q, k, v, out or row_max since, it runs the saved-statistics
 * backward (zt_attn_backward_train_ws on the holder's workspace, reading the
 * forward's scores on the first backward after that forward;
 * zt_attn_backward_train without a workspace); row_del receives
 * delta = sum_d out * dout.  Otherwise (no forward yet, a decode-shaped
 * forward_at, an upload, zt_holder_forget, or a holder from
 * zt_holder_init_exact) it runs zt_attn_backward, which rebuilds the
 * statistics into row_max / row_den / row_del as the reference does.  dq, dk,
 * dv agree between the two to rounding (same gates against the CPU twin). */
int zt_holder_backward(const zt_holder *h, int max_tile);
/* Drops the forward's saved state (no reference counterpart): the next
 * backward rebuilds the statistics. */
void zt_holder_forget(const zt_holder *h);
/* :412-431: bounds-checked against the target buffer's real byte count.  An
 * upload into q, k, v, out or row_max drops the forward's saved state. */
int zt_holder_upload(const zt_holder *h, int which, const float *src, size_t n_floats);
int zt_holder_download(const zt_holder *h, float *dst, int which, size_t n_floats);

#ifdef __cplusplus
}
#endif
#endif
