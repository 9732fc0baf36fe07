// The reference's device.Attn holder (src/cuda/device.zig:119-501) restated in
// C++ over the zt_attn C ABI.  Same checks in the same order, same five errors.
// One deliberate difference: a failed hipMemcpy is DeviceTransferFailed, the
// error device.zig:134-140 documents for it (its upload/download at :418,:430
// return DeviceAllocFailed instead).
//
// Saved statistics.  device.zig:400-402 requires the forward to have run on the
// same buffers before the backward, so the holder keeps what its forward
// formed instead of making the backward rebuild it: a whole-cache forward runs
// zt_attn_forward_train_ws (log-sum-exp into row_max, 1.0 into row_den, so
// p = exp(s - row_max) / row_den still holds, and the scores into a workspace
// the holder owns), and the next backward runs zt_attn_backward_train_ws
// reading them (row_del receives delta = sum_d out * dout).  The state is
// dropped by any upload into q, k, v, out or row_max, by a decode-shaped
// forward_at, and by zt_holder_forget; a backward without a current forward
// runs the reference pair (zt_attn_backward), which rebuilds the statistics.
// The workspace is taken at the first whole-shape forward (a holder that only
// decodes never takes it).  Without it (its allocation failed, it would take
// more than a quarter of the device's free memory, or zt_holder_init_exact)
// the fast pair is zt_attn_forward_train + zt_attn_backward_train.
//
// One query row.  device.zig's forwardAt with t = 1 is the reference's decode
// seam (src/decode.zig:462): one sequence, so the one-row forward of
// zt_attn_forward has only (kv head x head sub-group) workgroups and cannot
// fill the device.  The holder owns a small partials buffer (allocated at
// init, zt_attn_decode_workspace bytes for one sequence of t rows) and runs
// zt_attn_decode instead, which splits the visible keys into chunks across
// the device and merges the chunk partials.
#include <hip/hip_runtime_api.h>

#include <climits>
#include <cstdint>
#include <new>

#include "../../include/zt_attn.h"
#include "../../include/zt_holder.h"

namespace zt {

static bool mul_ok(size_t a, size_t b, size_t *out) {
    if (a != 0 && b > SIZE_MAX / a) return false;
    *out = a * b;
    return true;
}

int bytes_for(int kind, size_t t, size_t n_heads, size_t n_kv_heads, size_t dim, size_t *out) {
    if (t == 0 || dim == 0 || n_heads == 0 || n_kv_heads == 0) return ZT_DEGENERATE_SHAPE;
    size_t cols = 0;
    switch (kind) {
    case ZT_QUERY_HEADED:
        if (!mul_ok(n_heads, dim, &cols)) return ZT_SHAPE_TOO_LARGE;
        break;
    case ZT_KV_HEADED:
        if (!mul_ok(n_kv_heads, dim, &cols)) return ZT_SHAPE_TOO_LARGE;
        break;
    case ZT_PER_ROW:
        cols = n_heads;
        break;
    default:
        return ZT_CONFIG_REFUSED;
    }
    size_t elems = 0;
    if (!mul_ok(t, cols, &elems)) return ZT_SHAPE_TOO_LARGE;
    if (!mul_ok(elems, sizeof(float), out)) return ZT_SHAPE_TOO_LARGE;
    return ZT_OK;
}

int to_cint(size_t x, int *out) {
    if (x > (size_t)INT_MAX) return ZT_SHAPE_TOO_LARGE;
    *out = (int)x;
    return ZT_OK;
}

int forward_bounds(int c_t, int q_offset, int n_keys, int t) {
    if (n_keys < 1 || n_keys > c_t) return ZT_SHAPE_TOO_LARGE;
    if (t < 1 || t > c_t) return ZT_SHAPE_TOO_LARGE;
    if (q_offset < 0 || q_offset > c_t || t > c_t - q_offset) return ZT_SHAPE_TOO_LARGE;
    if (q_offset + t > n_keys) return ZT_SHAPE_TOO_LARGE;
    return ZT_OK;
}

// What the last forward left for the backward.
enum class Saved { None, Lse, Scores };

struct Attn {
    float *buf[ZT_N_BUFFERS] = {};
    size_t t = 0, n_heads = 0, n_kv_heads = 0, dim = 0;
    int c_t = 0, c_heads = 0, c_kv_heads = 0, c_dim = 0;
    void *ws = nullptr;  // zt_attn_backward_train_workspace bytes, or null
    size_t ws_bytes = 0;
    void *dec_ws = nullptr;  // zt_attn_decode_workspace bytes for one sequence, or null
    size_t dec_bytes = 0;
    bool fast = true;    // false: the reference pair only (zt_holder_init_exact)
    mutable bool ws_tried = false;  // the first whole-shape forward has asked for the score workspace
    mutable Saved saved = Saved::None;

    // The score workspace, asked for once (by the first whole-shape forward).
    // It is an optimisation: without it the holder still runs the
    // saved-statistics pair, so a failed allocation is no error.  It grows
    // with t^2 (1.0 GiB at t = 4096 with 32 heads, 4.0 GiB at 8192), so it is
    // taken only while it stays within a quarter of the device's free memory,
    // leaving the rest to the caller.
    void take_workspace() const {
        if (ws_tried) return;
        ws_tried = true;
        const size_t wsb = zt_attn_backward_train_workspace(1, c_t, c_heads, c_kv_heads, c_dim);
        size_t free_b = 0, total_b = 0;
        const bool fits = hipMemGetInfo(&free_b, &total_b) == hipSuccess && wsb <= free_b / 4;
        void *p = nullptr;
        if (wsb != 0 && fits && hipMalloc(&p, wsb) == hipSuccess && p) {
            Attn *self = const_cast<Attn *>(this);
            self->ws = p;
            self->ws_bytes = wsb;
        } else {
            (void)hipGetLastError();
        }
    }

    size_t buffer_bytes(int which) const {
        size_t n = 0;
        const int kind = (which == ZT_BUF_Q || which == ZT_BUF_OUT || which == ZT_BUF_DOUT || which == ZT_BUF_DQ)
                             ? ZT_QUERY_HEADED
                             : (which >= ZT_BUF_ROW_MAX ? ZT_PER_ROW : ZT_KV_HEADED);
        if (bytes_for(kind, t, n_heads, n_kv_heads, dim, &n) != ZT_OK) return 0;
        return n;
    }
    void free_taken(int taken) {
        for (int i = 0; i < taken; ++i) {
            if (buf[i]) (void)hipFree(buf[i]);
            buf[i] = nullptr;
        }
        if (ws) (void)hipFree(ws);
        ws = nullptr;
        ws_bytes = 0;
        if (dec_ws) (void)hipFree(dec_ws);
        dec_ws = nullptr;
        dec_bytes = 0;
    }
};

// The reference forward's own admission of group_q and max_tile
// (src/cuda/attn_kernels.cu:858-871): the fast forward ignores both, so it is
// taken only for arguments the reference entry point would accept too.
static bool forward_args_ok(int group_q, int max_tile, int dim) {
    return group_q >= 1 && group_q <= 64 && (size_t)dim * (size_t)group_q <= 1024 && max_tile >= 1;
}

}  // namespace zt

struct zt_holder {
    zt::Attn a;
};

extern "C" {

int zt_bytes_for(int kind, size_t t, size_t n_heads, size_t n_kv_heads, size_t dim, size_t *out) {
    return zt::bytes_for(kind, t, n_heads, n_kv_heads, dim, out);
}

int zt_to_cint(size_t x, int *out) { return zt::to_cint(x, out); }

int zt_forward_bounds(int c_t, int q_offset, int n_keys, int t) {
    return zt::forward_bounds(c_t, q_offset, n_keys, t);
}

static int holder_init(size_t t, size_t n_heads, size_t n_kv_heads, size_t dim, bool fast, zt_holder **out) {
    if (!out) return ZT_CONFIG_REFUSED;
    *out = nullptr;
    int c_t, c_heads, c_kv, c_dim, e;
    if ((e = zt::to_cint(t, &c_t)) || (e = zt::to_cint(n_heads, &c_heads)) || (e = zt::to_cint(n_kv_heads, &c_kv)) ||
        (e = zt::to_cint(dim, &c_dim)))
        return e;
    if (zt_attn_dim_ok(c_dim) == 0) return ZT_CONFIG_REFUSED;
    if (c_heads <= 0 || c_kv <= 0 || c_heads % c_kv != 0) return ZT_CONFIG_REFUSED;
    if (n_heads > 65535) return ZT_CONFIG_REFUSED;
    size_t qh, kvh, pr;
    if ((e = zt::bytes_for(ZT_QUERY_HEADED, t, n_heads, n_kv_heads, dim, &qh)) ||
        (e = zt::bytes_for(ZT_KV_HEADED, t, n_heads, n_kv_heads, dim, &kvh)) ||
        (e = zt::bytes_for(ZT_PER_ROW, t, n_heads, n_kv_heads, dim, &pr)))
        return e;
    zt_holder *h = new (std::nothrow) zt_holder;
    if (!h) return ZT_DEVICE_ALLOC_FAILED;
    const size_t sizes[ZT_N_BUFFERS] = {qh, kvh, kvh, qh, qh, qh, kvh, kvh, pr, pr, pr};
    for (int i = 0; i < ZT_N_BUFFERS; ++i) {
        void *p = nullptr;
        if (hipMalloc(&p, sizes[i]) != hipSuccess || !p) {
            (void)hipGetLastError();
            h->a.free_taken(i);
            delete h;
            return ZT_DEVICE_ALLOC_FAILED;
        }
        h->a.buf[i] = static_cast<float *>(p);
    }
    h->a.t = t; h->a.n_heads = n_heads; h->a.n_kv_heads = n_kv_heads; h->a.dim = dim;
    h->a.c_t = c_t; h->a.c_heads = c_heads; h->a.c_kv_heads = c_kv; h->a.c_dim = c_dim;
    h->a.fast = fast;
    if (fast) {
        // The one-row forward's chunk partials (about 1 MiB at t = 8192 with 32
        // heads); without them forward_at(t = 1) takes zt_attn_forward, so a
        // failed allocation is no error.  (The score workspace is taken by the
        // first whole-shape forward: a decode-only holder never needs it.)
        const size_t decb = zt_attn_decode_workspace(1, c_t, c_heads, c_kv, c_dim);
        void *p = nullptr;
        if (decb != 0 && hipMalloc(&p, decb) == hipSuccess && p) {
            h->a.dec_ws = p;
            h->a.dec_bytes = decb;
        } else {
            (void)hipGetLastError();
        }
    }
    *out = h;
    return ZT_OK;
}

int zt_holder_init(size_t t, size_t n_heads, size_t n_kv_heads, size_t dim, zt_holder **out) {
    return holder_init(t, n_heads, n_kv_heads, dim, true, out);
}

int zt_holder_init_exact(size_t t, size_t n_heads, size_t n_kv_heads, size_t dim, zt_holder **out) {
    return holder_init(t, n_heads, n_kv_heads, dim, false, out);
}

size_t zt_holder_workspace_bytes(const zt_holder *h) { return h ? h->a.ws_bytes + h->a.dec_bytes : 0; }

void zt_holder_forget(const zt_holder *h) {
    if (h) h->a.saved = zt::Saved::None;
}

void zt_holder_deinit(zt_holder *h) {
    if (!h) return;
    h->a.free_taken(ZT_N_BUFFERS);
    delete h;
}

size_t zt_holder_total_bytes(const zt_holder *h) {
    size_t qh = 0, kvh = 0, pr = 0;
    if (zt::bytes_for(ZT_QUERY_HEADED, h->a.t, h->a.n_heads, h->a.n_kv_heads, h->a.dim, &qh) ||
        zt::bytes_for(ZT_KV_HEADED, h->a.t, h->a.n_heads, h->a.n_kv_heads, h->a.dim, &kvh) ||
        zt::bytes_for(ZT_PER_ROW, h->a.t, h->a.n_heads, h->a.n_kv_heads, h->a.dim, &pr))
        return 0;
    return 4 * qh + 4 * kvh + 3 * pr;
}

float *zt_holder_buffer(const zt_holder *h, int which) {
    if (!h || which < 0 || which >= ZT_N_BUFFERS) return nullptr;
    // A writable pointer to an input of the saved state: the caller may change
    // what the forward saw, so the next backward rebuilds the statistics.
    if (which == ZT_BUF_Q || which == ZT_BUF_K || which == ZT_BUF_V || which == ZT_BUF_OUT || which == ZT_BUF_ROW_MAX)
        h->a.saved = zt::Saved::None;
    return h->a.buf[which];
}

const float *zt_holder_buffer_ro(const zt_holder *h, int which) {
    if (!h || which < 0 || which >= ZT_N_BUFFERS) return nullptr;
    return h->a.buf[which];
}

int zt_holder_forward_at(const zt_holder *h, int group_q, int max_tile, int q_offset, int n_keys, int t) {
    const zt::Attn &a = h->a;
    if (int e = zt::forward_bounds(a.c_t, q_offset, n_keys, t)) return e;
    a.saved = zt::Saved::None;
    const bool whole = q_offset == 0 && n_keys == a.c_t && t == a.c_t;
    if (a.fast && whole && zt::forward_args_ok(group_q, max_tile, a.c_dim)) {
        a.take_workspace();
        float *lse = a.buf[ZT_BUF_ROW_MAX];
        const int rc = a.ws ? zt_attn_forward_train_ws(a.buf[ZT_BUF_Q], a.buf[ZT_BUF_K], a.buf[ZT_BUF_V],
                                                       a.buf[ZT_BUF_OUT], lse, a.ws, a.ws_bytes, 1, a.c_t, a.c_heads,
                                                       a.c_kv_heads, a.c_dim, nullptr)
                            : zt_attn_forward_train(a.buf[ZT_BUF_Q], a.buf[ZT_BUF_K], a.buf[ZT_BUF_V],
                                                    a.buf[ZT_BUF_OUT], lse, 1, a.c_t, a.c_heads, a.c_kv_heads,
                                                    a.c_dim, nullptr);
        if (rc != 0) return ZT_CONFIG_REFUSED;
        // row_den = 1: with row_max = lse, p = exp(s - row_max) / row_den is the softmax.
        if (hipMemsetD32Async(a.buf[ZT_BUF_ROW_DEN], 0x3f800000, (size_t)a.c_t * (size_t)a.c_heads, nullptr) !=
            hipSuccess) {
            (void)hipGetLastError();
            return ZT_CONFIG_REFUSED;
        }
        a.saved = a.ws ? zt::Saved::Scores : zt::Saved::Lse;
        return ZT_OK;
    }
    if (a.dec_ws && t == 1 && zt::forward_args_ok(group_q, max_tile, a.c_dim)) {
        // The query at q_offset sees keys 0..q_offset (q_offset + 1 <= n_keys by
        // forward_bounds): the split-K decode over those rows of the holder's cache.
        const int visible = q_offset + 1;
        const int rc = zt_attn_decode(a.buf[ZT_BUF_Q], a.buf[ZT_BUF_K], a.buf[ZT_BUF_V], a.buf[ZT_BUF_OUT], &visible,
                                      1, a.c_t, a.c_heads, a.c_kv_heads, a.c_dim, a.dec_ws, a.dec_bytes, nullptr);
        return rc != 0 ? ZT_CONFIG_REFUSED : ZT_OK;
    }
    const int rc = zt_attn_forward(a.buf[ZT_BUF_Q], a.buf[ZT_BUF_K], a.buf[ZT_BUF_V], a.buf[ZT_BUF_OUT], t, a.c_heads,
                                   a.c_kv_heads, a.c_dim, group_q, max_tile, q_offset, n_keys, nullptr);
    return rc != 0 ? ZT_CONFIG_REFUSED : ZT_OK;
}

int zt_holder_forward(const zt_holder *h, int group_q, int max_tile) {
    return zt_holder_forward_at(h, group_q, max_tile, 0, h->a.c_t, h->a.c_t);
}

int zt_holder_backward(const zt_holder *h, int max_tile) {
    const zt::Attn &a = h->a;
    if (a.saved != zt::Saved::None && max_tile >= 1) {
        float *row_del = a.buf[ZT_BUF_ROW_DEL];
        const size_t per_row = (size_t)a.c_t * (size_t)a.c_heads;
        int rc;
        if (a.ws) {
            rc = zt_attn_backward_train_ws(a.buf[ZT_BUF_Q], a.buf[ZT_BUF_K], a.buf[ZT_BUF_V], a.buf[ZT_BUF_OUT],
                                           a.buf[ZT_BUF_DOUT], a.buf[ZT_BUF_ROW_MAX], a.buf[ZT_BUF_DQ],
                                           a.buf[ZT_BUF_DK], a.buf[ZT_BUF_DV], a.ws, a.ws_bytes, 1, a.c_t, a.c_heads,
                                           a.c_kv_heads, a.c_dim, a.saved == zt::Saved::Scores ? 3 | ZT_WS_SCORES : 3,
                                           nullptr);
            // delta sits at the workspace's start; row_del keeps the reference's scratch contract.
            if (rc == 0 && hipMemcpyAsync(row_del, a.ws, per_row * sizeof(float), hipMemcpyDeviceToDevice, nullptr) !=
                               hipSuccess) {
                (void)hipGetLastError();
                rc = 1;
            }
        } else {
            rc = zt_attn_backward_train(a.buf[ZT_BUF_Q], a.buf[ZT_BUF_K], a.buf[ZT_BUF_V], a.buf[ZT_BUF_OUT],
                                        a.buf[ZT_BUF_DOUT], a.buf[ZT_BUF_ROW_MAX], a.buf[ZT_BUF_DQ], a.buf[ZT_BUF_DK],
                                        a.buf[ZT_BUF_DV], row_del, 1, a.c_t, a.c_heads, a.c_kv_heads, a.c_dim,
                                        nullptr);
        }
        // The score tiles now hold dS: a second backward rebuilds them from lse.
        a.saved = zt::Saved::Lse;
        return rc != 0 ? ZT_CONFIG_REFUSED : ZT_OK;
    }
    const int rc = zt_attn_backward(a.buf[ZT_BUF_Q], a.buf[ZT_BUF_K], a.buf[ZT_BUF_V], a.buf[ZT_BUF_DOUT],
                                    a.buf[ZT_BUF_DQ], a.buf[ZT_BUF_DK], a.buf[ZT_BUF_DV], a.buf[ZT_BUF_ROW_MAX],
                                    a.buf[ZT_BUF_ROW_DEN], a.buf[ZT_BUF_ROW_DEL], a.c_t, a.c_heads, a.c_kv_heads,
                                    a.c_dim, max_tile, nullptr);
    return rc != 0 ? ZT_CONFIG_REFUSED : ZT_OK;
}

int zt_holder_upload(const zt_holder *h, int which, const float *src, size_t n_floats) {
    if (!h || which < 0 || which >= ZT_N_BUFFERS) return ZT_CONFIG_REFUSED;
    size_t n = 0;
    if (!zt::mul_ok(n_floats, sizeof(float), &n)) return ZT_SHAPE_TOO_LARGE;
    if (n > h->a.buffer_bytes(which)) return ZT_SHAPE_TOO_LARGE;
    // New q, k, v, out or lse: the forward's saved state no longer describes them.
    if (which == ZT_BUF_Q || which == ZT_BUF_K || which == ZT_BUF_V || which == ZT_BUF_OUT || which == ZT_BUF_ROW_MAX)
        h->a.saved = zt::Saved::None;
    if (hipMemcpy(h->a.buf[which], src, n, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipGetLastError();
        return ZT_DEVICE_TRANSFER_FAILED;
    }
    return ZT_OK;
}

int zt_holder_download(const zt_holder *h, float *dst, int which, size_t n_floats) {
    if (!h || which < 0 || which >= ZT_N_BUFFERS) return ZT_CONFIG_REFUSED;
    size_t n = 0;
    if (!zt::mul_ok(n_floats, sizeof(float), &n)) return ZT_SHAPE_TOO_LARGE;
    if (n > h->a.buffer_bytes(which)) return ZT_SHAPE_TOO_LARGE;
    if (hipMemcpy(dst, h->a.buf[which], n, hipMemcpyDeviceToHost) != hipSuccess) {
        (void)hipGetLastError();
        return ZT_DEVICE_TRANSFER_FAILED;
    }
    return ZT_OK;
}

}  // extern "C"
