// Host side of libzt_attn.so: validation, tile choice and kernel launch.
//
// The gfx950 code objects (kernels/*.hip built with --genco) are embedded in
// this library and loaded per device with hipModuleLoadData on first use;
// kernels are launched with hipModuleLaunchKernel, each taking one argument
// block (kernels/args.h).  There is one code path per operation and no CPU
// fallback: without a usable device every launcher refuses.
//
// Validation follows the reference launchers' order and return convention
// (src/cuda/attn_kernels.cu:833-1036): 0 = launch accepted, 1 = refused with
// the reason on stderr.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <initializer_list>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/zt_attn.h"
#include "kernels/args.h"

extern "C" {
extern const unsigned char zt_co_fwd[], zt_co_fwd_end[];
extern const unsigned char zt_co_bwd[], zt_co_bwd_end[];
extern const unsigned char zt_co_dec[], zt_co_dec_end[];
extern const unsigned char zt_co_misc[], zt_co_misc_end[];
extern const unsigned char zt_co_cal[], zt_co_cal_end[];
extern const unsigned char zt_co_gemm[], zt_co_gemm_end[];
int zt_noalloc_scratch_address(void **ptr);  // noalloc.hip
}

namespace {

constexpr int kMinDim = 32, kMaxDim = ZT_MAX_DIM;
constexpr int kMaxDevices = 64;
constexpr int kThreads = 256;

struct DeviceState {
    std::once_flag once;
    bool ok = false;
    size_t lds_limit = 0;
    int cus = 0;
    hipModule_t mods[6] = {};
    float *scratch = nullptr;  // this device's address of noalloc.hip's scratch (null: unavailable)
    std::mutex mu;
    std::unordered_map<std::string, hipFunction_t> fns;
};
DeviceState g_dev[kMaxDevices];

// Kernels live in the code object named by their prefix; a lookup never
// touches another module, so no failed hipModuleGetFunction is left behind in
// the thread's last-error slot for the caller's next HIP call to report.
int module_of(const char *name) {
    if (strncmp(name, "zt_fwd", 6) == 0) return 0;
    if (strncmp(name, "zt_bwd", 6) == 0) return 1;
    if (strncmp(name, "zt_dec", 6) == 0) return 2;
    if (strncmp(name, "zt_cal", 6) == 0) return 4;
    if (strncmp(name, "zt_gem", 6) == 0) return 5;
    return 3;
}

// A kernel's handle, from the cache or the code object (cached then); the
// caller holds st.mu, or is load_device (before any other thread sees st).
hipFunction_t resolve_fn(DeviceState &st, const char *name) {
    auto it = st.fns.find(name);
    if (it != st.fns.end()) return it->second;
    hipFunction_t f = nullptr;
    if (hipModuleGetFunction(&f, st.mods[module_of(name)], name) != hipSuccess || !f) {
        (void)hipGetLastError();
        return nullptr;
    }
    st.fns.emplace(name, f);
    return f;
}

void load_device(DeviceState &st, int dev) {
    int lds = 0;
    if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || lds <= 0)
        return;
    const unsigned char *images[6] = {zt_co_fwd, zt_co_bwd, zt_co_dec, zt_co_misc, zt_co_cal, zt_co_gemm};
    for (int i = 0; i < 6; ++i) {
        if (hipModuleLoadData(&st.mods[i], images[i]) != hipSuccess) {
            fprintf(stderr, "zt_attn: the gfx950 code object %d would not load on device %d.\n", i, dev);
            return;
        }
    }
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 1;
    st.cus = cus;
    st.lds_limit = (size_t)lds;
    // The no-allocation decode's scratch: its address on this device, asked
    // once while the device is current (each device holds its own copy).
    void *scratch = nullptr;
    if (zt_noalloc_scratch_address(&scratch) == 0) st.scratch = static_cast<float *>(scratch);
    // The decode kernels' handles, resolved now so that a later
    // zt_attn_decode_noalloc (possibly under graph capture) only looks them up.
    char name[32];
    for (int dp : {32, 64, 128, 256}) {
        for (int g : {1, 2, 4, 8}) {
            snprintf(name, sizeof name, "zt_dec_d%d_g%d", dp, g);
            resolve_fn(st, name);
        }
        for (int g : {1, 2}) {
            snprintf(name, sizeof name, "zt_dec8_d%d_g%d", dp, g);
            resolve_fn(st, name);
        }
    }
    for (const char *c : {"v16", "v32", "v64", "s64", "s128", "s256"}) {
        snprintf(name, sizeof name, "zt_dec_combine_%s", c);
        resolve_fn(st, name);
    }
    st.ok = true;
}

// The current device's state, code objects loaded; nullptr when there is no
// usable device (which every launcher reads as a refusal).
DeviceState *device_state() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        return nullptr;
    }
    DeviceState &st = g_dev[dev];
    std::call_once(st.once, load_device, std::ref(st), dev);
    return st.ok ? &st : nullptr;
}

hipFunction_t get_fn(DeviceState *st, const char *name) {
    std::lock_guard<std::mutex> lk(st->mu);
    return resolve_fn(*st, name);
}


template <class Args>
int launch(DeviceState *st, const char *name, unsigned blocks, const Args &args, hipStream_t stream,
           unsigned threads = kThreads) {
    hipFunction_t f = get_fn(st, name);
    if (!f) {
        fprintf(stderr, "zt_attn: FAIL kernel %s is missing from the code object.\n", name);
        return 1;
    }
    Args copy = args;
    void *params[] = {&copy};
    const hipError_t e = hipModuleLaunchKernel(f, blocks, 1, 1, threads, 1, 1, 0, stream, params, nullptr);
    if (e != hipSuccess) {
        fprintf(stderr, "zt_attn: FAIL launch of %s: %s\n", name, hipGetErrorString(e));
        return 1;
    }
    return 0;
}

// Tuning variables: every kernel variant is chosen from the shape unless one of
// these is set, which happens only through zt_attn_set_tuning (sweeps and the
// tests that force each variant).  The process environment is never read, so
// nothing outside the caller's own calls changes which kernel runs.  A plain
// array of atomics: the launchers read it without a lock.
enum Tune {
    kTuneBK, kTuneFwdW, kTuneFPF, kTuneFPair, kTuneQPF, kTuneDqW, kTuneHS, kTuneW8, kTunePF, kTuneDMA, kTuneBPair,
    kTuneDSplit, kTuneRSplit, kTuneDecWgs, kTuneGemmTile, kTuneGemmSk, kTuneGemmSkTile, kTuneDqdsTile, kTuneRowG,
    kTuneRowW, kTuneFKS, kTuneDqdsK, kTuneRScores, kTuneCount
};
struct TuneSpec {
    const char *name;
    int allowed[10];
    int n_allowed;
};
const TuneSpec kTuneSpecs[kTuneCount] = {
    {"ZT_ATTN_BK", {32, 64}, 2},
    {"ZT_ATTN_FWD_W", {4, 8}, 2},
    {"ZT_ATTN_FPF", {0, 1}, 2},
    {"ZT_ATTN_FPAIR", {0, 1}, 2},
    {"ZT_ATTN_QPF", {0, 1}, 2},
    {"ZT_ATTN_DQ_W", {4, 8}, 2},
    {"ZT_ATTN_HS", {1, 2, 4}, 3},
    {"ZT_ATTN_W8", {0, 1}, 2},
    {"ZT_ATTN_PF", {0, 1}, 2},
    {"ZT_ATTN_DMA", {0, 1}, 2},
    {"ZT_ATTN_BPAIR", {0, 1}, 2},
    {"ZT_ATTN_DSPLIT", {0, 1}, 2},
    {"ZT_ATTN_RSPLIT", {0, 1}, 2},
    {"ZT_DEC_WGS", {256, 512, 768, 1024, 1536, 2048, 4096, 8192, 16384, 32768}, 10},
    {"ZT_GEMM_TILE", {32, 64, 128}, 3},
    {"ZT_GEMM_SK", {0, 4, 8, 16}, 4},
    {"ZT_GEMM_SK_TILE", {16, 32}, 2},
    {"ZT_DQDS_TILE", {64, 128}, 2},
    {"ZT_ROW_G", {1, 2, 4, 8}, 4},
    {"ZT_ROW_W", {4, 8}, 2},
    {"ZT_ATTN_FKS", {1, 2}, 2},
    {"ZT_DQDS_K", {1, 2}, 2},
    {"ZT_ATTN_RSCORES", {0, 1}, 2},
};
std::atomic<int> g_tune[kTuneCount] = {};  // 0 = unset (no allowed value is 0 except a flag, stored as value + 1)

// The forced value of a variable, or `dflt` (the shape rule) when unset.
int tuned(Tune id, int dflt) {
    const int v = g_tune[id].load(std::memory_order_relaxed);
    return v == 0 ? dflt : v - 1;
}

int pad32(int dim) { return (dim + 31) / 32 * 32; }

int heads_per_wg(int group) { return group % 4 == 0 ? 4 : (group % 2 == 0 ? 2 : 1); }

// Key tile (keys staged in LDS per step) for a width and a caller cap: 64 or
// 32.  Measured on MI355X (C2/C3/C5 shapes): the dq kernel takes 32 keys with
// the next tile prefetched into registers (C3 2.43 -> 2.23 ms, C2 0.132 ->
// 0.119 ms, C5 1.74 -> 1.65 ms against 64 keys without); so does the forward
// wherever rows are 16-byte chunks (dim % 4 == 0; C2 0.074 -> 0.057 ms), and
// without the prefetch it prefers 64 only at d <= 64 -- above that the 32-key
// tile keeps one more workgroup resident per CU (C5, d = 256: 0.84 ms vs 1.11 ms).
enum class Tiled { Forward, Dq };
int key_tile(Tiled which, int dp, int max_tile, int dim = 0) {
    const int dflt = (which == Tiled::Forward && dp <= 64 && dim % 4 != 0) ? 64 : 32;
    const int preferred = tuned(kTuneBK, dflt);
    return max_tile >= 64 ? preferred : 32;
}
// LDS per workgroup: K and V tiles, row-major with a 4-float pad.
size_t fwd_tile_bytes(int dp, int bk) { return (size_t)2 * bk * (dp + 4) * sizeof(float); }
size_t kv_tile_bytes(int dp, int bk) { return (size_t)2 * bk * (dp + 4) * sizeof(float); }

// Waves per forward / dq workgroup (4 or 8): eight waves share each staged K/V
// tile between twice as many query rows.  Measured on MI355X: the forward
// gains when four query heads share a kv group (C3 1.39 -> 1.33 ms, C5 0.84 ->
// 0.76 ms) and, with the register prefetch, when two do (B = 4, T = 2048, 16
// heads over 8, d = 128: 0.647 -> 0.581 ms; d = 256, B = 2: 0.711 -> 0.588 ms);
// it loses for MHA (C2 0.057 -> 0.076 ms); the dq kernel loses at every shape tried.
int fwd_waves(int hw) { return tuned(kTuneFwdW, hw >= 2 ? 8 : 4); }

// Forward kernel name: waves per workgroup, key tile, and for 32-key tiles the
// register-prefetched variant (ZT_ATTN_FPF=0 turns it off).  Measured on
// MI355X: eight waves, C3 1.315 -> 1.225 ms and C5 0.758 -> 0.630 ms; four
// waves (MHA and head groups of two), C2 0.074 -> 0.057 ms and one 16-head
// sequence of 2048 rows at d = 128 0.30 -> 0.185 ms.
void fwd_kernel_name(char *name, size_t len, int dim, int dp, int bk, int nw, int ks = 1) {
    // The prefetching kernels load 16-byte row chunks unconditionally (dim % 4 == 0).
    const bool pf = bk == 32 && dim % 4 == 0 && tuned(kTuneFPF, 1) == 1;
    if (pf && ks > 1)
        snprintf(name, len, "zt_fwdpk_d%d_k32", dp);
    else if (pf)
        snprintf(name, len, nw == 8 ? "zt_fwd8p_d%d_k32" : "zt_fwdp_d%d_k32", dp);
    else
        snprintf(name, len, nw == 8 ? "zt_fwd8_d%d_k%d" : "zt_fwd_d%d_k%d", dp, bk);
}

// Key parts of the forward: 1, or 2 for the key-split kernel (zt_fwdpk_*:
// eight waves, 4 row blocks x 2 key parts merged at the end) for one query
// head per workgroup (HW = 1) where the four-wave kernel's grid, after
// pairing, gives at most one workgroup per CU: one wave per SIMD there, and
// the split doubles it for the same rows.  Measured on MI355X (training
// forward): C2 60.8 -> 51.3 us, one 16-head sequence of 2048 rows at d = 64
// 104.5 -> 85.5 us, 12 heads of 1024 rows at d = 128, B = 2, 94.9 -> 89.5 us.
// Needs the prefetching kernel (32-key tiles, dim % 4 == 0) and d <= 128.
int fwd_key_split(int B, int T, int n_heads, int hw, int dp, int dim, int bk, int cus) {
    const bool able = hw == 1 && dp <= 128 && bk == 32 && dim % 4 == 0 && tuned(kTuneFPF, 1) == 1;
    const long long tiles = (T + 63) / 64;  // 64-row tiles (4 row blocks) per head
    const long long wgs = (tiles + 1) / 2 * (long long)n_heads * B;  // paired
    return able ? tuned(kTuneFKS, wgs <= cus ? 2 : 1) : 1;
}
int dq_waves(int dp) {
    const int w = tuned(kTuneDqW, 4);
    return dp > 192 ? 4 : w;  // eight-wave dq spills above d = 192
}
// bufs: stage buffers (2 in the register-prefetching kernels).
size_t dkdv_bytes(int dp, int hs, int kw = 0, int rows = 16, int bufs = 1) {
    if (kw == 0) kw = 4 / hs;
    const size_t stage = ((size_t)2 * hs * rows * (dp + 4) + (size_t)hs * rows * 4) * bufs;
    const size_t red = (size_t)(hs - 1) * kw * 64 * 2 * (dp / 16) * 4;
    return (stage > red ? stage : red) * sizeof(float);
}
// The asynchronously staged dk/dv kernel: two buffers of unpadded tiles.
size_t dkdv_dma_bytes(int dp, int hs) { return ((size_t)2 * hs * 2 * 16 * dp + (size_t)2 * hs * 16 * 4) * sizeof(float); }
// The column-split score-reading kernel (d = 192, 256): two 16-row stage
// buffers for two head halves plus the partial-dP exchange of its eight waves.
size_t dkdv_ds_bytes(int dp) { return dkdv_bytes(dp, 2, 2, 16, 2) + (size_t)8 * 64 * 4 * sizeof(float); }
// The same for the kernel that forms S again: partial S and dP exchanged
// (hs 1: one part of four key blocks).
size_t dkdv_dspd_bytes(int dp, int hs = 2) {
    return dkdv_bytes(dp, hs, 4 / hs, 16, 2) + (size_t)2 * 8 * 64 * 4 * sizeof(float);
}
// Score-reading dk/dv kernel for heads wider than 128: the column-split
// eight-wave kernel where the head halves are whole 32-column groups (two
// waves per SIMD instead of one), else the four-wave asynchronously staged
// one.  ZT_ATTN_DSPLIT=0 forces the latter.
// Paired tiles (forward rows, dk/dv keys) by default only when the unpaired grid is larger than the CU count.
int pair_pays(unsigned long long unpaired_blocks, int cus) { return unpaired_blocks > (unsigned long long)cus ? 1 : 0; }
bool dkdv_dsplit(int dp, size_t lds_limit) {
    return (dp == 192 || dp == 256) && dkdv_ds_bytes(dp) <= lds_limit && tuned(kTuneDSplit, 1) == 1;
}

int refuse_T(int T) {
    fprintf(stderr,
            "zt_attn: T %d is not launchable. A zero or negative query count\n"
            "       gives a grid with no workgroups.\n",
            T);
    return 1;
}

int refuse_dim(int dim) {
    fprintf(stderr, "zt_attn: head_dim %d is refused. It must be even and in [%d, %d].\n", dim, kMinDim, kMaxDim);
    return 1;
}

int check_group(int n_heads, int n_kv_heads) {
    if (n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0) {
        fprintf(stderr, "zt_attn: %d heads over %d kv heads is not a group.\n", n_heads, n_kv_heads);
        return 1;
    }
    if (n_heads > 65535) {
        fprintf(stderr, "zt_attn: %d heads exceeds the 65535 head limit.\n", n_heads);
        return 1;
    }
    return 0;
}

int refuse_max_tile(int max_tile) {
    fprintf(stderr, "zt_attn: max_tile %d is not launchable. A tile of zero never advances the key loop.\n",
            max_tile);
    return 1;
}

DeviceState *require_device() {
    DeviceState *st = device_state();
    if (!st) {
        fprintf(stderr, "zt_attn: this device's LDS ceiling could not be read (no usable gfx950 device or code\n"
                        "       object), so no tile can be sized against it. Refusing rather than guessing.\n");
    }
    return st;
}

// The launch's total work-items (workgroups x threads per workgroup) must fit
// HIP's 32-bit grid.
bool grid_ok(unsigned long long blocks, unsigned threads = kThreads) {
    if (blocks == 0 || blocks * threads > 0xFFFFFFFFull) {
        fprintf(stderr, "zt_attn: the launch would need %llu workgroups, beyond the 2^32 work-item grid.\n", blocks);
        return false;
    }
    return true;
}

static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Workspaces hold 16-byte vectors (tiles, partials) at 256-byte aligned
// offsets from their base, so the base must be 16-byte aligned (hipMalloc
// returns 256).
static bool workspace_aligned(const void *ws, const char *who) {
    if ((uintptr_t)ws & 15) {
        fprintf(stderr, "zt_attn: %s workspace at %p is not 16-byte aligned.\n", who, ws);
        return false;
    }
    return true;
}

// Rows are read with 16-byte vector loads when dim % 4 == 0 and with 8-byte
// loads otherwise, so every tensor base (null ones aside) must be aligned to that.
static bool rows_aligned(int dim, std::initializer_list<const void *> ptrs) {
    const uintptr_t mask = (dim & 3) == 0 ? 15 : 7;
    for (const void *p : ptrs) {
        if (p && ((uintptr_t)p & mask)) {
            fprintf(stderr, "zt_attn: tensor at %p is not %d-byte aligned, as head_dim %d rows need.\n", p,
                    (int)mask + 1, dim);
            return false;
        }
    }
    return true;
}

// One query row per sequence (T = 1: a decode step through the reference entry
// point, src/decode.zig:462, whose query at position q_offset sees the first
// n_vis = q_offset + 1 keys): the decode kernel with the whole visible prefix in
// one chunk per (sequence, kv head, head sub-group), so each workgroup writes
// `out` itself and no workspace is needed.  Measured on MI355X (C4's 64
// sequences of 8192 keys, 32 / 8 heads, d = 128, one call per sequence): the
// forward kernel took 665 us per call, 15 of every 16 rows of its MFMA tiles
// idle; the decode kernel with four query heads per workgroup (8 workgroups)
// 319 us, with one (32 workgroups, each kv head's rows read four times, the
// repeats from cache) 237 us, and with eight waves per workgroup 143 us.
// Without a workspace the key axis cannot be split, so a single sequence has
// only H / G workgroups: where they cannot fill the device, G = 1 and eight
// waves.
// The one-row forward's head sub-group G, waves per workgroup and kernel name.
void one_row_plan(const DeviceState *st, int B, int n_heads, int n_kv_heads, int dim, int *G_out, int *nw_out,
                  char *name, size_t len) {
    const int group = n_heads / n_kv_heads;
    const int dp = dim <= 32 ? 32 : dim <= 64 ? 64 : dim <= 128 ? 128 : 256;
    const int g_fill = group % 8 == 0 ? 8 : group % 4 == 0 ? 4 : group % 2 == 0 ? 2 : 1;
    const bool few = (unsigned long long)B * n_kv_heads * (group / g_fill) < (unsigned long long)st->cus;
    int G = tuned(kTuneRowG, few ? 1 : g_fill);
    if (group % G != 0) G = 1;
    int nw = tuned(kTuneRowW, few ? 8 : 4);
    if (G > 2) nw = 4;  // eight waves instantiated for one or two heads per workgroup
    snprintf(name, len, nw == 8 ? "zt_dec8_d%d_g%d" : "zt_dec_d%d_g%d", dp, G);
    *G_out = G;
    *nw_out = nw;
}

int forward_one_row(DeviceState *st, const float *q, const float *k, const float *v, float *out, int B, int n_heads,
                    int n_kv_heads, int dim, int n_vis, int kv_rows, hipStream_t stream) {
    int G = 0, nw = 0;
    char name[64];
    one_row_plan(st, B, n_heads, n_kv_heads, dim, &G, &nw, name, sizeof name);
    const int n_gsub = n_heads / n_kv_heads / G;
    DecArgs a{};
    a.q = q; a.kc = k; a.vc = v; a.out = out;
    a.part_acc = nullptr; a.part_ml = nullptr;  // one chunk: never touched
    a.n_ctx = kv_rows; a.H = n_heads; a.Hkv = n_kv_heads; a.dim = dim;
    a.chunk = n_vis; a.n_chunks = 1; a.n_gsub = n_gsub;
    a.scale_log2e = (float)(1.4426950408889634 / std::sqrt((double)dim));
    for (int b0 = 0; b0 < B; b0 += ZT_DEC_MAXB) {
        a.b_base = b0;
        a.nb = B - b0 < ZT_DEC_MAXB ? B - b0 : ZT_DEC_MAXB;
        for (int i = 0; i < a.nb; ++i) a.n_keys[i] = n_vis;
        const unsigned long long blocks = (unsigned long long)a.nb * n_kv_heads * n_gsub;
        if (!grid_ok(blocks, 64u * nw)) return 1;
        if (launch(st, name, (unsigned)blocks, a, stream, 64u * nw)) return 1;
    }
    return 0;
}

int forward_impl(const float *q, const float *k, const float *v, float *out, int B, int T, int n_heads,
                 int n_kv_heads, int dim, int group_q, int max_tile, int q_offset, int n_keys, int kv_rows,
                 hipStream_t stream, float *lse = nullptr, float *s_out = nullptr) {
    if (T < 1) return refuse_T(T);
    if (!zt_attn_dim_ok(dim)) return refuse_dim(dim);
    if (check_group(n_heads, n_kv_heads)) return 1;
    if (group_q < 1 || group_q > 64 || (size_t)dim * (size_t)group_q > 1024) {
        fprintf(stderr, "zt_attn: group_q %d at head_dim %d is not launchable.\n", group_q, dim);
        return 1;
    }
    if (q_offset < 0 || n_keys < 1 || q_offset > n_keys - T) {
        fprintf(stderr, "zt_attn: q_offset %d, n_keys %d is not launchable.\n", q_offset, n_keys);
        return 1;
    }
    if (max_tile < 1) return refuse_max_tile(max_tile);
    if (B < 1 || kv_rows < n_keys) {
        fprintf(stderr, "zt_attn: batch %d with %d kv rows per sequence (n_keys %d) is not launchable.\n", B,
                kv_rows, n_keys);
        return 1;
    }
    DeviceState *st = require_device();
    if (!st) return 1;
    if (T == 1 && !lse && !s_out) {
        if (!q || !k || !v || !out) {
            fprintf(stderr, "zt_attn: a null tensor pointer is not launchable.\n");
            return 1;
        }
        if (!rows_aligned(dim, {q, k, v, out})) return 1;
        return forward_one_row(st, q, k, v, out, B, n_heads, n_kv_heads, dim, q_offset + 1, kv_rows, stream);
    }
    const int dp = pad32(dim);
    int bk = key_tile(Tiled::Forward, dp, max_tile, dim);
    if (fwd_tile_bytes(dp, bk) > st->lds_limit) bk = 32;
    if (fwd_tile_bytes(dp, bk) > st->lds_limit) {
        fprintf(stderr, "zt_attn: head_dim %d needs %zu bytes of LDS per workgroup even at a 32-key tile, and\n"
                        "       this device grants %zu. Refusing.\n",
                dim, fwd_tile_bytes(dp, bk), st->lds_limit);
        return 1;
    }
    if (!q || !k || !v || !out) {
        fprintf(stderr, "zt_attn: a null tensor pointer is not launchable.\n");
        return 1;
    }
    if (!rows_aligned(dim, {q, k, v, out})) return 1;
    FwdArgs a{};
    a.q = q; a.k = k; a.v = v; a.out = out; a.lse = lse; a.s_out = s_out;
    a.B = B; a.T = T; a.H = n_heads; a.Hkv = n_kv_heads; a.dim = dim;
    a.q_offset = q_offset; a.n_keys = n_keys; a.kv_rows = kv_rows;
    a.HW = heads_per_wg(n_heads / n_kv_heads);
    const int ks = fwd_key_split(B, T, n_heads, a.HW, dp, dim, bk, st->cus);
    const int nw = ks > 1 ? 8 : fwd_waves(a.HW);
    const int rows_per_wg = 16 * (nw / ks / a.HW);
    a.n_row_tiles = (T + rows_per_wg - 1) / rows_per_wg;
    a.n_head_blocks = n_heads / a.HW;
    a.scale_log2e = (float)(1.4426950408889634 / std::sqrt((double)dim));
    // Paired row tiles (n - 1 - p, then p): equal causal work per workgroup;
    // measured on MI355X, C3 1.22 -> 1.13 ms, C5 0.63 -> 0.61 ms, C2 0.082 -> 0.072 ms.
    // Not when the unpaired grid fits the CUs once (one MHA sequence, T 1024,
    // d 64: 0.070 -> 0.064 ms without).
    a.pair = tuned(kTuneFPair, pair_pays((unsigned long long)a.n_row_tiles * a.n_head_blocks * B, st->cus));
    const unsigned long long blocks =
        (unsigned long long)(a.pair ? (a.n_row_tiles + 1) / 2 : a.n_row_tiles) * a.n_head_blocks * B;
    if (!grid_ok(blocks, 64u * nw)) return 1;
    char name[64];
    fwd_kernel_name(name, sizeof name, dim, dp, bk, nw, ks);
    if (s_out && dp <= 128 && strncmp(name, "zt_fwd8p_d", 10) == 0)
        snprintf(name, sizeof name, "zt_fwd8ps_d%d_k32", dp);  // same kernel, named for its role
    return launch(st, name, (unsigned)blocks, a, stream, 64u * nw);
}

// Validates a backward call and fills the argument block and kernel names.
// Returns 0 when launchable; prints the refusal and returns 1 otherwise.
int backward_prepare(const float *q, const float *k, const float *v, const float *dout, float *dq, float *dk,
                     float *dv, float *row_max, float *row_den, float *row_del, int B, int T, int n_heads,
                     int n_kv_heads, int dim, int max_tile, BwdArgs *a, DeviceState **st_out, char *name_dq,
                     char *name_dkdv, unsigned *blocks_dq, unsigned *blocks_dkdv, unsigned *threads_dq,
                     unsigned *threads_dkdv, const float *o = nullptr, const float *lse = nullptr) {
    const bool saved = lse != nullptr;  // statistics from the forward: 32-key, four-wave dq kernel
    if (T < 1) return refuse_T(T);
    if (!zt_attn_dim_ok(dim)) return refuse_dim(dim);
    if (check_group(n_heads, n_kv_heads)) return 1;
    if (max_tile < 1) return refuse_max_tile(max_tile);
    if (B < 1) {
        fprintf(stderr, "zt_attn: batch %d is not launchable.\n", B);
        return 1;
    }
    DeviceState *st = require_device();
    if (!st) return 1;
    const int dp = pad32(dim);
    int bk = saved ? 32 : key_tile(Tiled::Dq, dp, max_tile);
    if (kv_tile_bytes(dp, bk) > st->lds_limit) bk = 32;
    const int group = n_heads / n_kv_heads;
    // dk/dv head split: two parts where the group allows (measured best at
    // g = 4, d = 128 and 256: half the Q/dO staging of a 4-way split, twice
    // the workgroups of none).
    const int hs_dflt = group % 2 == 0 ? 2 : 1;
    int hs = tuned(kTuneHS, hs_dflt);
    if (group % hs != 0 || (hs == 4 && dp > 128)) hs = hs_dflt;  // 4-way split instantiated up to d = 128
    while (hs > 1 && dkdv_bytes(dp, hs) > st->lds_limit) hs /= 2;
    if (kv_tile_bytes(dp, bk) > st->lds_limit || dkdv_bytes(dp, hs) > st->lds_limit) {
        fprintf(stderr, "zt_attn: head_dim %d needs more LDS per workgroup than this device grants (%zu).\n", dim,
                st->lds_limit);
        return 1;
    }
    if (!q || !k || !v || !dout || !row_max || !row_den || !row_del || (!dq && !dk && !dv)) {
        fprintf(stderr, "zt_attn: a null tensor pointer is not launchable.\n");
        return 1;
    }
    if (saved && !o) {
        fprintf(stderr, "zt_attn: the saved-statistics backward needs the forward output.\n");
        return 1;
    }
    if (!rows_aligned(dim, {q, k, v, dout, dq, dk, dv, o})) return 1;
    *a = BwdArgs{};
    a->o = o; a->lse = lse;
    a->q = q; a->k = k; a->v = v; a->dout = dout;
    a->dq = dq; a->dk = dk; a->dv = dv;
    a->row_max = row_max; a->row_den = row_den; a->row_del = row_del;
    a->B = B; a->T = T; a->H = n_heads; a->Hkv = n_kv_heads; a->dim = dim;
    a->HW = heads_per_wg(group);
    const int nw_dq = saved ? 4 : dq_waves(dp);
    const int rows_per_wg = 16 * (nw_dq / a->HW);
    a->n_row_tiles = (T + rows_per_wg - 1) / rows_per_wg;
    a->n_head_blocks = n_heads / a->HW;
    a->HS = hs;
    // dk/dv variant, measured on MI355X (C2/C3/C5 shapes):
    //  - eight-wave workgroups (4 key blocks x 2 head halves share each staged
    //    Q/dO tile) for a 2-way split up to d = 128 (C3: 2.91 ms vs 3.22 ms);
    //  - d = 192, 256: eight waves splitting the head's columns in two, two
    //    per SIMD (C5: 1.32 ms vs 1.57 ms for the kernel below);
    //  - asynchronous double-buffered staging for the other wide heads (C5
    //    before the column split: 1.97 ms vs 2.27 ms) and for grids too small
    //    to hide the staging latency with other workgroups; it needs
    //    whole-head rows on 16-byte aligned q/dout;
    //  - otherwise the four-wave register-staged kernel.
    const bool wide = tuned(kTuneW8, 1) == 1 && hs == 2 && dp <= 128 &&
                      dkdv_bytes(dp, 2, 4) <= st->lds_limit;
    const int keys_per_wg = wide ? 64 : 16 * (4 / hs);
    a->n_key_tiles = (T + keys_per_wg - 1) / keys_per_wg;
    // Paired tiles (a workgroup takes tile p and its partner n - 1 - p): equal
    // causal work per workgroup; measured on MI355X, C3 dk/dv 2.47 -> 2.37 ms,
    // reading scores 2.01 -> 1.93 ms, C5 1.49 -> 1.43 ms.  Not when the
    // unpaired grid already fits the CUs once: pairing would leave CUs idle
    // (one MHA sequence, T 1024, d 64: 0.131 -> 0.122 ms without).
    a->pair = tuned(kTuneBPair, pair_pays((unsigned long long)a->n_key_tiles * n_kv_heads * B, st->cus));
    const unsigned long long blocks_b =
        (unsigned long long)(a->pair ? (a->n_key_tiles + 1) / 2 : a->n_key_tiles) * n_kv_heads * B;
    const bool aligned = ((uintptr_t)q % 16 == 0) && ((uintptr_t)dout % 16 == 0);
    const bool dma_ok = dim == dp && aligned && !(hs == 4 && dp > 128) && !(hs == 1 && dp >= 224) &&
                        dkdv_dma_bytes(dp, hs) <= st->lds_limit;
    // Asynchronous staging pays where at most one workgroup per CU runs (C2:
    // 0.165 -> 0.137 ms) and for wide heads.
    const bool dma_pays =
        dp >= 160 || (unsigned long long)((a->n_key_tiles + 1) / 2) * n_kv_heads * B <= (unsigned long long)st->cus;
    const bool dma_want = tuned(kTuneDMA, dma_pays ? 1 : 0) == 1;
    // Eight waves splitting the head's columns in two (two waves per SIMD)
    // where the halves are whole 32-column groups: at d = 192, 256 instead of
    // the four-wave kernels (C5 and the reference entry points); for a group
    // that cannot be halved (MHA, odd groups) also at d = 64, 128 where the
    // asynchronously staged kernel is not chosen (MHA, d = 128, B = 2, T = 2048:
    // 1.13 -> 0.72 ms; d = 64, B = 8, T = 1024: 0.90 -> 0.80 ms; where that
    // kernel is chosen it stays ahead, C2 0.105 ms against 0.125 ms).
    // ZT_ATTN_DSPLIT=0 turns it off.
    const bool dsplit = !wide && hs <= 2 && dim == dp && aligned && dkdv_dspd_bytes(dp, hs) <= st->lds_limit &&
                        (dp == 192 || dp == 256 || (hs == 1 && (dp == 64 || dp == 128) && !dma_want)) &&
                        tuned(kTuneDSplit, 1) == 1;
    const bool dma = !wide && !dsplit && dma_ok && dma_want;
    // A group that cannot be split (MHA, odd groups) on the asynchronously
    // staged kernel: two row parts per workgroup instead, eight waves.
    const bool rsplit = dma && hs == 1 && dp <= 128 && dkdv_dma_bytes(dp, 2) <= st->lds_limit &&
                        tuned(kTuneRSplit, 1) == 1;
    a->scale = (float)(1.0 / std::sqrt((double)dim));
    a->scale_log2e = (float)(1.4426950408889634 / std::sqrt((double)dim));
    const unsigned long long blocks_a =
        (unsigned long long)(a->pair ? (a->n_row_tiles + 1) / 2 : a->n_row_tiles) * a->n_head_blocks * B;
    const bool qpf = bk == 32 && tuned(kTuneQPF, 1) == 1;
    if (saved)
        snprintf(name_dq, 64, "zt_bwd_dql_d%d_k32", dp);
    else if (qpf)
        snprintf(name_dq, 64, nw_dq == 8 ? "zt_bwd_dq8p_d%d_k32" : "zt_bwd_dqp_d%d_k32", dp);
    else
        snprintf(name_dq, 64, nw_dq == 8 ? "zt_bwd_dq8_d%d_k%d" : "zt_bwd_dq_d%d_k%d", dp, bk);
    *threads_dq = 64u * nw_dq;
    // The prefetching kernel loads whole 16-byte chunks unconditionally.
    const bool pf = dim % 4 == 0 && aligned && dkdv_bytes(dp, 2, 4, 16, 2) <= st->lds_limit &&
                    tuned(kTunePF, 1) == 1;
    if (wide)
        snprintf(name_dkdv, 64, pf ? "zt_bwd_dkdv8p_d%d_hs2" : "zt_bwd_dkdv8_d%d_hs2", dp);
    else if (dsplit)
        snprintf(name_dkdv, 64, "zt_bwd_dkdv8pd_d%d_hs%d", dp, hs);
    else if (rsplit)
        snprintf(name_dkdv, 64, "zt_bwd_dkdv_dmar_d%d", dp);
    else
        snprintf(name_dkdv, 64, dma ? "zt_bwd_dkdv_dma_d%d_hs%d" : "zt_bwd_dkdv_d%d_hs%d", dp, hs);
    *threads_dkdv = wide || dsplit || rsplit ? 512 : kThreads;
    if (!grid_ok(blocks_a, *threads_dq) || !grid_ok(blocks_b, *threads_dkdv)) return 1;
    *blocks_dq = (unsigned)blocks_a;
    *blocks_dkdv = (unsigned)blocks_b;
    *st_out = st;
    return 0;
}

// stage: 1 = dq + row statistics, 2 = dk/dv (reads the statistics), 3 = both.
int backward_impl(const float *q, const float *k, const float *v, const float *dout, float *dq, float *dk,
                  float *dv, float *row_max, float *row_den, float *row_del, int B, int T, int n_heads,
                  int n_kv_heads, int dim, int max_tile, int stage, hipStream_t stream, const float *o = nullptr,
                  const float *lse = nullptr) {
    BwdArgs a;
    DeviceState *st = nullptr;
    char name_a[64], name_b[64];
    unsigned blocks_a = 0, blocks_b = 0, threads_a = kThreads, threads_b = kThreads;
    if (backward_prepare(q, k, v, dout, dq, dk, dv, row_max, row_den, row_del, B, T, n_heads, n_kv_heads, dim,
                         max_tile, &a, &st, name_a, name_b, &blocks_a, &blocks_b, &threads_a, &threads_b, o, lse))
        return 1;
    if ((stage & 1) && !dq) {
        fprintf(stderr, "zt_attn: a null dq is not launchable.\n");
        return 1;
    }
    if ((stage & 2) && (!dk || !dv)) {
        fprintf(stderr, "zt_attn: a null dk or dv is not launchable.\n");
        return 1;
    }
    if ((stage & 1) && launch(st, name_a, blocks_a, a, stream, threads_a)) return 1;
    // Same stream: the dk/dv kernel reads the row statistics the first wrote.
    if ((stage & 2) && launch(st, name_b, blocks_b, a, stream, threads_b)) return 1;
    return 0;
}

// Decode geometry: head sub-group G, padded width, keys per step and chunk.
struct DecGeom {
    int G, n_gsub, dp, ks, chunk, n_chunks;
};

DecGeom decode_geom(int B, int n_ctx, int n_heads, int n_kv_heads, int dim) {
    DecGeom g{};
    const int group = n_heads / n_kv_heads;
    g.G = group % 8 == 0 ? 8 : group % 4 == 0 ? 4 : group % 2 == 0 ? 2 : 1;
    g.n_gsub = group / g.G;
    g.dp = dim <= 32 ? 32 : dim <= 64 ? 64 : dim <= 128 ? 128 : 256;
    g.ks = 4 * (64 / (g.dp / 4));  // the kernel's step: 4 loads of 64 / (dp / 4) rows
    const long long pairs = (long long)B * n_kv_heads * g.n_gsub;
    // Workgroups to aim for: 512, two per CU of MI355X's 256 (the workspace
    // size must not depend on the device). Measured on MI355X against 1024 / 2048
    // (C4 643 -> 624 us; B = 1, 8192 keys 66 -> 41 us; B = 16, 4096 keys 106 -> 93 us).
    const long long target = tuned(kTuneDecWgs, 512);
    long long per_seq = (target + pairs - 1) / pairs;
    if (per_seq < 1) per_seq = 1;
    long long chunk = (n_ctx + per_seq - 1) / per_seq;
    const long long gran = 8LL * g.ks;  // every wave of four gets at least its two buffers' steps
    chunk = (chunk + gran - 1) / gran * gran;
    if (chunk < gran) chunk = gran;
    g.chunk = (int)chunk;
    g.n_chunks = (int)((n_ctx + chunk - 1) / chunk);
    return g;
}

}  // namespace

extern "C" {

int zt_attn_dim_ok(int dim) { return !(dim < kMinDim || dim > kMaxDim || (dim & 1) != 0); }

size_t zt_attn_forward_shmem(int dim, int tile, int group_q) {
    (void)group_q;
    if (!zt_attn_dim_ok(dim)) return 0;
    const int dp = pad32(dim);
    return fwd_tile_bytes(dp, key_tile(Tiled::Forward, dp, tile, dim));
}

size_t zt_attn_bwd_dq_shmem(int dim, int tile) {
    if (!zt_attn_dim_ok(dim)) return 0;
    const int dp = pad32(dim);
    return kv_tile_bytes(dp, key_tile(Tiled::Dq, dp, tile));
}

size_t zt_attn_bwd_dkdv_shmem(int dim) {
    if (!zt_attn_dim_ok(dim)) return 0;
    const int dp = pad32(dim);
    size_t most = dkdv_bytes(dp, dp <= 128 ? 4 : 2);
    if (dp <= 128) most = std::max(most, dkdv_bytes(dp, 2, 4, 32, 2));  // eight waves, two 32-row stage buffers
    if (dp == 192 || dp == 256)  // column-split eight waves
        most = std::max(most, std::max(dkdv_dspd_bytes(dp, 2), dkdv_dspd_bytes(dp, 1)));
    if (dp == 64 || dp == 128) most = std::max(most, dkdv_dspd_bytes(dp, 1));
    for (int hs : {1, 2, 4})
        if (!(hs == 4 && dp > 128) && dkdv_dma_bytes(dp, hs) > most) most = dkdv_dma_bytes(dp, hs);
    return most;
}

int zt_attn_forward(const float *q, const float *k, const float *v, float *out, int T, int n_heads,
                    int n_kv_heads, int dim, int group_q, int max_tile, int q_offset, int n_keys,
                    hipStream_t stream) {
    return forward_impl(q, k, v, out, 1, T, n_heads, n_kv_heads, dim, group_q, max_tile, q_offset, n_keys,
                        n_keys, stream);
}

int zt_attn_forward_batched(const float *q, const float *k, const float *v, float *out, int B, int T,
                            int n_heads, int n_kv_heads, int dim, int group_q, int max_tile, int q_offset,
                            int n_keys, int kv_rows, hipStream_t stream) {
    return forward_impl(q, k, v, out, B, T, n_heads, n_kv_heads, dim, group_q, max_tile, q_offset, n_keys,
                        kv_rows, stream);
}

int zt_attn_backward(const float *q, const float *k, const float *v, const float *dout, float *dq, float *dk,
                     float *dv, float *row_max, float *row_den, float *row_del, int T, int n_heads,
                     int n_kv_heads, int dim, int max_tile, hipStream_t stream) {
    return backward_impl(q, k, v, dout, dq, dk, dv, row_max, row_den, row_del, 1, T, n_heads, n_kv_heads, dim,
                         max_tile, 3, stream);
}

int zt_attn_backward_batched(const float *q, const float *k, const float *v, const float *dout, float *dq,
                             float *dk, float *dv, float *row_max, float *row_den, float *row_del, int B, int T,
                             int n_heads, int n_kv_heads, int dim, int max_tile, hipStream_t stream) {
    return backward_impl(q, k, v, dout, dq, dk, dv, row_max, row_den, row_del, B, T, n_heads, n_kv_heads, dim,
                         max_tile, 3, stream);
}

int zt_attn_forward_train(const float *q, const float *k, const float *v, float *out, float *lse, int B, int T,
                          int n_heads, int n_kv_heads, int dim, hipStream_t stream) {
    if (!lse && T >= 1 && zt_attn_dim_ok(dim)) {
        fprintf(stderr, "zt_attn: forward_train needs an lse buffer.\n");
        return 1;
    }
    return forward_impl(q, k, v, out, B, T, n_heads, n_kv_heads, dim, 1, 64, 0, T, T, stream, lse);
}

static int train_stats_ok(const float *lse, const float *delta) {
    if (!lse || !delta) {
        fprintf(stderr, "zt_attn: the saved-statistics backward needs lse and a delta buffer.\n");
        return 0;
    }
    return 1;
}

int zt_attn_backward_train(const float *q, const float *k, const float *v, const float *out, const float *dout,
                           const float *lse, float *dq, float *dk, float *dv, float *delta, int B, int T,
                           int n_heads, int n_kv_heads, int dim, hipStream_t stream) {
    if (!train_stats_ok(lse, delta)) return 1;
    float *l = const_cast<float *>(lse);  // read only in this mode
    return backward_impl(q, k, v, dout, dq, dk, dv, l, l, delta, B, T, n_heads, n_kv_heads, dim, 64, 3, stream, out,
                         lse);
}

int zt_attn_bwd_dq_train(const float *q, const float *k, const float *v, const float *out, const float *dout,
                         const float *lse, float *dq, float *delta, int B, int T, int n_heads, int n_kv_heads,
                         int dim, hipStream_t stream) {
    if (!train_stats_ok(lse, delta)) return 1;
    float *l = const_cast<float *>(lse);
    return backward_impl(q, k, v, dout, dq, nullptr, nullptr, l, l, delta, B, T, n_heads, n_kv_heads, dim, 64, 1,
                         stream, out, lse);
}

int zt_attn_bwd_dkdv_train(const float *q, const float *k, const float *v, const float *out, const float *dout,
                           const float *lse, const float *delta, float *dk, float *dv, int B, int T, int n_heads,
                           int n_kv_heads, int dim, hipStream_t stream) {
    if (!train_stats_ok(lse, delta)) return 1;
    float *l = const_cast<float *>(lse);
    return backward_impl(q, k, v, dout, nullptr, dk, dv, l, l, const_cast<float *>(delta), B, T, n_heads, n_kv_heads,
                         dim, 64, 2, stream, out, lse);
}

// Tile of the dq-from-dS product: 128 x 128 unless the head is 64 wide or less
// or 128-tiles would leave CUs idle.
static int dqds_tile(int B, int T, int n_heads, int dim, int cus) {
    const unsigned long long wgs128 =
        (unsigned long long)(((T + 127) / 128 + 1) / 2) * ((dim + 127) / 128) * B * n_heads;  // row-tile pairs
    return tuned(kTuneDqdsTile, (dim > 64 && wgs128 >= (unsigned long long)cus) ? 128 : 64);
}

// Key parts of the dq-from-dS product: 2 (zt_gemm_dqds2_*: eight waves, two
// four-wave parts taking alternate key slabs, their tiles added at the end)
// where the four-wave grid gives at most one workgroup per CU (one wave per
// SIMD), else 1.  The split kernels take 16-byte k rows (vec).
static int dqds_parts(int B, int T, int n_heads, int dim, int bt, bool vec, int cus) {
    const unsigned long long wgs = (unsigned long long)(((T + bt - 1) / bt + 1) / 2) * ((dim + bt - 1) / bt) * B * n_heads;
    return vec ? tuned(kTuneDqdsK, wgs <= (unsigned long long)cus ? 2 : 1) : 1;
}
static void dqds_name(char *name, size_t len, int bt, int parts) {
    snprintf(name, len, parts > 1 ? "zt_gemm_dqds2_%d" : "zt_gemm_dqds_%d", bt);
}

size_t zt_attn_backward_train_workspace(int B, int T, int n_heads, int n_kv_heads, int dim) {
    if (B < 1 || T < 1 || !zt_attn_dim_ok(dim) || n_heads <= 0 || n_kv_heads <= 0 || n_heads % n_kv_heads != 0)
        return 0;
    const int nt = (T + 15) / 16;  // dS in 16 x 16 tiles, the causal ones only
    return align256((size_t)B * T * n_heads * sizeof(float)) +
           (size_t)B * n_heads * (size_t)zt_tri_count(nt) * 256 * sizeof(float);
}

// Which dk/dv kernel takes the forward's scores instead of rebuilding them,
// if any.  Split: an even head group (two-way head split) with 16-byte row
// chunks (d % 4 == 0): up to d = 128 the eight-wave kernel with 32 query rows
// per stage, above it the asynchronously staged kernel (whole-head rows: d a
// multiple of 32).  RowSplit: a group that cannot be halved (MHA, odd groups)
// where the statistics path takes the row-split asynchronously staged kernel
// (whole-head rows up to d = 128, at most one paired workgroup per CU): the
// same kernel reading the scores (ZT_ATTN_RSCORES=0 keeps it forming S
// again).  Measured on MI355X (training step, scores against none): C2
// 179.6 -> 171.8-177.9 us, one 16-head MHA sequence of 2048 rows at d = 128
// 582 -> 530 us, B = 2, T = 1024, 12 over 4 heads at d = 64 320 -> 291 us,
// one 8-head sequence of 1024 rows at d = 96 217 -> 202 us; the forward pays
// 4-5 us for its score stores at each.  The forward writes scores only for
// these.
enum class ScoreKernel { None, Split, RowSplit };
static ScoreKernel score_kernel(int B, int T, int dim, int n_heads, int n_kv_heads, const DeviceState *st) {
    const int dp = pad32(dim);
    if (n_kv_heads <= 0 || n_heads % n_kv_heads != 0 || dim % 4 != 0) return ScoreKernel::None;
    if ((n_heads / n_kv_heads) % 2 == 0) {
        const bool fits = dp <= 128 ? dkdv_bytes(dp, 2, 4, 32, 2) <= st->lds_limit
                                    : dim == dp && dkdv_dma_bytes(dp, 2) <= st->lds_limit;
        return fits ? ScoreKernel::Split : ScoreKernel::None;
    }
    // The statistics path's choice for this shape (backward_prepare, HS = 1).
    const unsigned long long tiles = (unsigned long long)(T + 63) / 64;
    const bool dma_pays = (tiles + 1) / 2 * n_kv_heads * B <= (unsigned long long)st->cus;
    const bool rsplit = dim == dp && dp <= 128 && dkdv_dma_bytes(dp, 2) <= st->lds_limit &&
                        tuned(kTuneDMA, dma_pays ? 1 : 0) == 1 && tuned(kTuneRSplit, 1) == 1;
    return rsplit && tuned(kTuneRScores, 1) == 1 ? ScoreKernel::RowSplit : ScoreKernel::None;
}
static bool scores_path(int B, int T, int dim, int n_heads, int n_kv_heads, const DeviceState *st) {
    return score_kernel(B, T, dim, n_heads, n_kv_heads, st) != ScoreKernel::None;
}

static float *ws_tiles(void *workspace, int B, int T, int n_heads) {
    return reinterpret_cast<float *>(static_cast<char *>(workspace) + align256((size_t)B * T * n_heads * sizeof(float)));
}

// Which workspaces hold scores, and of what.  zt_attn_forward_train_ws stamps
// the workspace it wrote scores into with the call's device, q, k and shape;
// the first backward stage 1 that consumes them (ZT_WS_SCORES) checks the
// stamp against its own arguments and removes it, and so does any stage 1
// that writes dS over the tiles without reading them.  A ZT_WS_SCORES call
// with no matching stamp is refused instead of reading tiles that hold dS,
// another shape's scores, or nothing.  Host-side only: no device read, so the
// calls stay asynchronous.  What it cannot see is q or k rewritten in place
// between the two calls (the same pointers, other values) -- a change that
// makes the forward's out and lse stale too.
struct ScoreStamp {
    int dev;
    const void *ws;
    const float *q, *k;
    int B, T, H, Hkv, dim;
};
std::mutex g_stamp_mu;
std::vector<ScoreStamp> g_stamps;

static int current_device() {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return -1;
    }
    return dev;
}

static void stamp_drop_locked(int dev, const void *ws) {
    g_stamps.erase(std::remove_if(g_stamps.begin(), g_stamps.end(),
                                  [&](const ScoreStamp &s) { return s.dev == dev && s.ws == ws; }),
                   g_stamps.end());
}

static void stamp_set(const ScoreStamp &s) {
    std::lock_guard<std::mutex> lk(g_stamp_mu);
    stamp_drop_locked(s.dev, s.ws);
    g_stamps.push_back(s);
}

static void stamp_drop(const void *ws) {
    const int dev = current_device();
    std::lock_guard<std::mutex> lk(g_stamp_mu);
    stamp_drop_locked(dev, ws);
}

// True (and the stamp consumed) when `ws` holds the scores of exactly this q, k and shape.
static bool stamp_take(const ScoreStamp &want) {
    std::lock_guard<std::mutex> lk(g_stamp_mu);
    for (auto it = g_stamps.begin(); it != g_stamps.end(); ++it) {
        if (it->dev != want.dev || it->ws != want.ws) continue;
        const bool same = it->q == want.q && it->k == want.k && it->B == want.B && it->T == want.T &&
                          it->H == want.H && it->Hkv == want.Hkv && it->dim == want.dim;
        if (same) g_stamps.erase(it);  // a refused call writes nothing: the scores stay usable
        return same;
    }
    return false;
}

int zt_attn_forward_train_ws(const float *q, const float *k, const float *v, float *out, float *lse, void *workspace,
                             size_t workspace_bytes, int B, int T, int n_heads, int n_kv_heads, int dim,
                             hipStream_t stream) {
    if (!lse && T >= 1 && zt_attn_dim_ok(dim)) {
        fprintf(stderr, "zt_attn: forward_train needs an lse buffer.\n");
        return 1;
    }
    const size_t need = zt_attn_backward_train_workspace(B, T, n_heads, n_kv_heads, dim);
    if (need != 0 && (!workspace || workspace_bytes < need)) {
        fprintf(stderr, "zt_attn: forward_train_ws workspace of %zu bytes is short of the %zu needed.\n",
                workspace_bytes, need);
        return 1;
    }
    if (need != 0 && !workspace_aligned(workspace, "forward_train_ws")) return 1;
    DeviceState *st = need ? device_state() : nullptr;
    float *s_out = (st && scores_path(B, T, dim, n_heads, n_kv_heads, st)) ? ws_tiles(workspace, B, T, n_heads)
                                                                                : nullptr;
    const int rc = forward_impl(q, k, v, out, B, T, n_heads, n_kv_heads, dim, 1, 64, 0, T, T, stream, lse, s_out);
    // (A refused call wrote nothing, so whatever stamp the workspace had still holds.)
    if (rc == 0 && s_out)
        stamp_set(ScoreStamp{current_device(), workspace, q, k, B, T, n_heads, n_kv_heads, dim});
    else if (rc == 0 && workspace)
        stamp_drop(workspace);
    return rc;
}

int zt_attn_backward_train_ws(const float *q, const float *k, const float *v, const float *out, const float *dout,
                              const float *lse, float *dq, float *dk, float *dv, void *workspace,
                              size_t workspace_bytes, int B, int T, int n_heads, int n_kv_heads, int dim, int stage,
                              hipStream_t stream) {
    const bool scores = (stage & 4) != 0;
    stage &= 3;
    if (stage < 1) {
        fprintf(stderr, "zt_attn: backward_train_ws stage %d is not 1, 2 or 3 (optionally | 4).\n", stage);
        return 1;
    }
    if (!lse || !out) {
        fprintf(stderr, "zt_attn: the saved-statistics backward needs lse and the forward output.\n");
        return 1;
    }
    const size_t need = zt_attn_backward_train_workspace(B, T, n_heads, n_kv_heads, dim);
    if (need != 0 && (!workspace || workspace_bytes < need)) {
        fprintf(stderr, "zt_attn: backward_train_ws workspace of %zu bytes is short of the %zu needed.\n",
                workspace_bytes, need);
        return 1;
    }
    if (need != 0 && !workspace_aligned(workspace, "backward_train_ws")) return 1;
    float *delta = static_cast<float *>(workspace);
    float *ds = need ? ws_tiles(workspace, B, T, n_heads) : nullptr;
    BwdArgs a;
    DeviceState *st = nullptr;
    char name_a[64], name_b[64];
    unsigned blocks_a = 0, blocks_b = 0, threads_a = kThreads, threads_b = kThreads;
    float *l = const_cast<float *>(lse);
    if (backward_prepare(q, k, v, dout, dq, dk, dv, l, l, delta, B, T, n_heads, n_kv_heads, dim, 64, &a, &st, name_a,
                         name_b, &blocks_a, &blocks_b, &threads_a, &threads_b, out, lse))
        return 1;
    if (((stage & 1) && (!dk || !dv)) || ((stage & 2) && !dq)) {
        fprintf(stderr, "zt_attn: a null gradient pointer is not launchable.\n");
        return 1;
    }
    a.ds_out = ds;
    const int dp = pad32(dim);
    const bool qd_aligned = (uintptr_t)q % 16 == 0 && (uintptr_t)dout % 16 == 0;
    const ScoreKernel sk = score_kernel(B, T, dim, n_heads, n_kv_heads, st);
    // (RowSplit reads them on the grid backward_prepare sized for the row-split kernel.)
    const bool read_scores = scores && (stage & 1) && sk != ScoreKernel::None && qd_aligned &&
                             (sk != ScoreKernel::RowSplit || strncmp(name_b, "zt_bwd_dkdv_dmar_d", 18) == 0);
    if (read_scores &&
        !stamp_take(ScoreStamp{current_device(), workspace, q, k, B, T, n_heads, n_kv_heads, dim})) {
        fprintf(stderr,
                "zt_attn: ZT_WS_SCORES, but this workspace holds no scores that zt_attn_forward_train_ws wrote for\n"
                "       these q, k and this shape (or a backward stage 1 has already replaced them with dS).\n"
                "       Refusing rather than reading stale tiles: run the forward again, or drop ZT_WS_SCORES.\n");
        return 1;
    }
    if (read_scores && sk == ScoreKernel::RowSplit) {
        // The row-split kernel the statistics path chose (backward_prepare
        // set its grid), reading the scores instead of forming Q K^T.
        snprintf(name_b, sizeof name_b, "zt_bwd_dkdv_dmars_d%d", dp);
    } else if (read_scores) {
        // The forward left the scores in the dS tiles: a kernel that reads
        // them, 2 head halves x 64 keys (eight waves, d <= 128) or x 32 keys
        // (wider heads: eight waves splitting the columns, or four waves with
        // asynchronous staging) per workgroup.  (Unaligned q / dout rows form
        // Q K^T again.)
        a.HS = 2;
        const int keys = dp <= 128 ? 64 : 32;
        const bool dsplit = dp > 128 && dkdv_dsplit(dp, st->lds_limit);
        a.n_key_tiles = (T + keys - 1) / keys;
        a.pair = tuned(kTuneBPair, pair_pays((unsigned long long)a.n_key_tiles * n_kv_heads * B, st->cus));
        const unsigned long long blocks =
            (unsigned long long)(a.pair ? (a.n_key_tiles + 1) / 2 : a.n_key_tiles) * n_kv_heads * B;
        threads_b = dp <= 128 || dsplit ? 512 : 256;
        if (!grid_ok(blocks, threads_b)) return 1;
        blocks_b = (unsigned)blocks;
        snprintf(name_b, sizeof name_b,
                 dp <= 128 ? "zt_bwd_dkdv8s_d%d_hs2" : dsplit ? "zt_bwd_dkdv8sd_d%d_hs2" : "zt_bwd_dkdv_dmas_d%d_hs2",
                 dp);
    }
    if (stage & 1) {
        // Stage 1 writes dS over the tiles: whatever scores they held are gone.
        if (!read_scores) stamp_drop(workspace);
        const unsigned long long rows = (unsigned long long)B * T * n_heads;
        if (!grid_ok((rows + 15) / 16)) return 1;
        if (launch(st, "zt_bwd_delta", (unsigned)((rows + 15) / 16), a, stream)) return 1;
        // Same stream: dk/dv reads delta, then writes dS for the product below.
        if (launch(st, name_b, blocks_b, a, stream, threads_b)) return 1;
    }
    if (stage & 2) {
        DqDsArgs g{};
        g.ds = ds; g.k = k; g.dq = dq;
        g.B = B; g.T = T; g.H = n_heads; g.Hkv = n_kv_heads; g.dim = dim;
        g.scale = a.scale;
        g.vec = dim % 4 == 0 && (uintptr_t)k % 16 == 0;
        const int bt = dqds_tile(B, T, n_heads, dim, st->cus);
        g.tiles_m = (T + bt - 1) / bt;
        g.tiles_n = (dim + bt - 1) / bt;
        const unsigned long long blocks = (unsigned long long)((g.tiles_m + 1) / 2) * g.tiles_n * B * n_heads;
        const int parts = dqds_parts(B, T, n_heads, dim, bt, g.vec, st->cus);
        char name[64];
        dqds_name(name, sizeof name, bt, parts);
        if (!grid_ok(blocks, 256u * parts)) return 1;
        if (launch(st, name, (unsigned)blocks, g, stream, 256u * parts)) return 1;
    }
    return 0;
}

int zt_attn_bwd_dq(const float *q, const float *k, const float *v, const float *dout, float *dq, float *row_max,
                   float *row_den, float *row_del, int B, int T, int n_heads, int n_kv_heads, int dim, int max_tile,
                   hipStream_t stream) {
    return backward_impl(q, k, v, dout, dq, nullptr, nullptr, row_max, row_den, row_del, B, T, n_heads, n_kv_heads,
                         dim, max_tile, 1, stream);
}

int zt_attn_bwd_dkdv(const float *q, const float *k, const float *v, const float *dout, float *dk, float *dv,
                     const float *row_max, const float *row_den, const float *row_del, int B, int T, int n_heads,
                     int n_kv_heads, int dim, hipStream_t stream) {
    return backward_impl(q, k, v, dout, nullptr, dk, dv, const_cast<float *>(row_max), const_cast<float *>(row_den),
                         const_cast<float *>(row_del), B, T, n_heads, n_kv_heads, dim, 64, 2, stream);
}


size_t zt_attn_decode_workspace(int B, int n_ctx, int n_heads, int n_kv_heads, int dim) {
    if (B < 1 || n_ctx < 1 || !zt_attn_dim_ok(dim) || n_heads <= 0 || n_kv_heads <= 0 ||
        n_heads % n_kv_heads != 0)
        return 0;
    const DecGeom g = decode_geom(B, n_ctx, n_heads, n_kv_heads, dim);
    return (size_t)B * n_heads * g.n_chunks * ((size_t)dim + 2) * sizeof(float);
}

// The decode's checks up to its workspace, shared by zt_attn_decode and
// zt_attn_decode_noalloc: 0 when the shape is launchable.
static int decode_check(const int *n_keys, int B, int n_ctx, int n_heads, int n_kv_heads, int dim) {
    if (B < 1 || n_ctx < 1) {
        fprintf(stderr, "zt_attn: decode over %d sequences of %d cached rows is not launchable.\n", B, n_ctx);
        return 1;
    }
    if (!zt_attn_dim_ok(dim)) return refuse_dim(dim);
    if (check_group(n_heads, n_kv_heads)) return 1;
    if (!n_keys) {
        fprintf(stderr, "zt_attn: decode needs the host n_keys array.\n");
        return 1;
    }
    for (int b = 0; b < B; ++b) {
        if (n_keys[b] < 1 || n_keys[b] > n_ctx) {
            fprintf(stderr, "zt_attn: sequence %d has n_keys %d, outside [1, %d].\n", b, n_keys[b], n_ctx);
            return 1;
        }
    }
    return 0;
}

// Launches the decode (and, with more than one chunk per sequence, the
// combine) with the chunk partials at `part` (only read or written when
// there is more than one chunk).
static int decode_launch(DeviceState *st, const float *q, const float *k_cache, const float *v_cache, float *out,
                         const int *n_keys, int B, int n_ctx, int n_heads, int n_kv_heads, int dim, float *part,
                         hipStream_t stream);

int zt_attn_decode(const float *q, const float *k_cache, const float *v_cache, float *out, const int *n_keys,
                   int B, int n_ctx, int n_heads, int n_kv_heads, int dim, void *workspace,
                   size_t workspace_bytes, hipStream_t stream) {
    if (decode_check(n_keys, B, n_ctx, n_heads, n_kv_heads, dim)) return 1;
    const size_t need = zt_attn_decode_workspace(B, n_ctx, n_heads, n_kv_heads, dim);
    if (!workspace || workspace_bytes < need) {
        fprintf(stderr, "zt_attn: decode workspace of %zu bytes is short of the %zu needed.\n", workspace_bytes,
                need);
        return 1;
    }
    if (!workspace_aligned(workspace, "decode")) return 1;
    if (!q || !k_cache || !v_cache || !out) {
        fprintf(stderr, "zt_attn: a null tensor pointer is not launchable.\n");
        return 1;
    }
    if (!rows_aligned(dim, {q, k_cache, v_cache, out})) return 1;
    DeviceState *st = require_device();
    if (!st) return 1;
    return decode_launch(st, q, k_cache, v_cache, out, n_keys, B, n_ctx, n_heads, n_kv_heads, dim,
                         static_cast<float *>(workspace), stream);
}

int zt_attn_decode_noalloc(const float *q, const float *k_cache, const float *v_cache, float *out, const int *n_keys,
                           int B, int n_ctx, int n_heads, int n_kv_heads, int dim, hipStream_t stream) {
    if (decode_check(n_keys, B, n_ctx, n_heads, n_kv_heads, dim)) return 1;
    // The partials are needed only when a sequence's keys are split into chunks.
    const DecGeom g = decode_geom(B, n_ctx, n_heads, n_kv_heads, dim);
    const size_t need = g.n_chunks > 1 ? zt_attn_decode_workspace(B, n_ctx, n_heads, n_kv_heads, dim) : 0;
    if (need > ZT_NOALLOC_SCRATCH_BYTES) {
        fprintf(stderr,
                "zt_attn: decode_noalloc of %d sequences x %d heads in %d key chunks needs %zu bytes of partials,\n"
                "       beyond the library's fixed %u-byte scratch. Use zt_attn_decode with a workspace.\n",
                B, n_heads, g.n_chunks, need, ZT_NOALLOC_SCRATCH_BYTES);
        return 1;
    }
    if (!q || !k_cache || !v_cache || !out) {
        fprintf(stderr, "zt_attn: a null tensor pointer is not launchable.\n");
        return 1;
    }
    if (!rows_aligned(dim, {q, k_cache, v_cache, out})) return 1;
    DeviceState *st = require_device();
    if (!st) return 1;
    if (!st->scratch) {
        fprintf(stderr, "zt_attn: decode_noalloc's scratch has no address on this device.\n");
        return 1;
    }
    return decode_launch(st, q, k_cache, v_cache, out, n_keys, B, n_ctx, n_heads, n_kv_heads, dim, st->scratch,
                         stream);
}

static int decode_launch(DeviceState *st, const float *q, const float *k_cache, const float *v_cache, float *out,
                         const int *n_keys, int B, int n_ctx, int n_heads, int n_kv_heads, int dim, float *part,
                         hipStream_t stream) {
    const DecGeom g = decode_geom(B, n_ctx, n_heads, n_kv_heads, dim);
    DecArgs a{};
    a.q = q; a.kc = k_cache; a.vc = v_cache; a.out = out;
    a.part_acc = part;
    a.part_ml = a.part_acc + (size_t)B * n_heads * g.n_chunks * dim;
    a.n_ctx = n_ctx; a.H = n_heads; a.Hkv = n_kv_heads; a.dim = dim;
    a.chunk = g.chunk; a.n_chunks = g.n_chunks; a.n_gsub = g.n_gsub;
    a.scale_log2e = (float)(1.4426950408889634 / std::sqrt((double)dim));
    char name[64], combine[64];
    snprintf(name, sizeof name, "zt_dec_d%d_g%d", g.dp, g.G);
    // The combine: float4 columns when rows are whole float4 (16-byte aligned
    // partial rows: d % 4 == 0), dp / 4 threads per row; else one float each.
    if (dim % 4 == 0)
        snprintf(combine, sizeof combine, "zt_dec_combine_v%d", g.dp <= 64 ? 16 : g.dp / 4);
    else
        snprintf(combine, sizeof combine, "zt_dec_combine_s%d", g.dp < 64 ? 64 : g.dp);
    for (int b0 = 0; b0 < B; b0 += ZT_DEC_MAXB) {
        a.b_base = b0;
        a.nb = B - b0 < ZT_DEC_MAXB ? B - b0 : ZT_DEC_MAXB;
        for (int i = 0; i < a.nb; ++i) a.n_keys[i] = n_keys[b0 + i];
        const unsigned long long blocks = (unsigned long long)a.nb * g.n_chunks * n_kv_heads * g.n_gsub;
        if (!grid_ok(blocks)) return 1;
        if (launch(st, name, (unsigned)blocks, a, stream)) return 1;
        // One chunk per sequence: the decode kernel wrote the output itself.
        if (g.n_chunks > 1 && launch(st, combine, (unsigned)(a.nb * n_heads), a, stream)) return 1;
    }
    return 0;
}

size_t zt_attn_decode_step_workspace(int B, int n_ctx, int n_heads, int n_kv_heads, int dim) {
    const size_t dec = zt_attn_decode_workspace(B, n_ctx, n_heads, n_kv_heads, dim);
    if (dec == 0) return 0;
    return align256(dec) + (size_t)B * n_heads * dim * sizeof(float);  // + the rotated queries
}

int zt_attn_decode_step(const float *q, const float *k_new, const float *v_new, float *k_cache, float *v_cache,
                        float *out, const int *pos, int B, int n_ctx, int n_heads, int n_kv_heads, int dim,
                        double theta, void *workspace, size_t workspace_bytes, hipStream_t stream) {
    if (B < 1 || n_ctx < 1) {
        fprintf(stderr, "zt_attn: decode over %d sequences of %d cached rows is not launchable.\n", B, n_ctx);
        return 1;
    }
    if (!zt_attn_dim_ok(dim)) return refuse_dim(dim);
    if (check_group(n_heads, n_kv_heads)) return 1;
    if (!pos) {
        fprintf(stderr, "zt_attn: decode_step needs the host pos array.\n");
        return 1;
    }
    for (int b = 0; b < B; ++b) {
        if (pos[b] < 0 || pos[b] >= n_ctx) {  // src/kv_cache.zig:88-95: a full cache refuses
            fprintf(stderr, "zt_attn: sequence %d appends at position %d, outside the %d-row cache.\n", b, pos[b],
                    n_ctx);
            return 1;
        }
    }
    if (!(theta > 0.0)) {
        fprintf(stderr, "zt_attn: RoPE theta %g is not usable.\n", theta);
        return 1;
    }
    const size_t need = zt_attn_decode_step_workspace(B, n_ctx, n_heads, n_kv_heads, dim);
    if (!workspace || workspace_bytes < need) {
        fprintf(stderr, "zt_attn: decode_step workspace of %zu bytes is short of the %zu needed.\n",
                workspace_bytes, need);
        return 1;
    }
    if (!workspace_aligned(workspace, "decode_step")) return 1;
    if (!q || !k_new || !v_new || !k_cache || !v_cache || !out) {
        fprintf(stderr, "zt_attn: a null tensor pointer is not launchable.\n");
        return 1;
    }
    if (!rows_aligned(dim, {k_cache, v_cache, out})) return 1;
    DeviceState *st = require_device();
    if (!st) return 1;
    const size_t dec_bytes = zt_attn_decode_workspace(B, n_ctx, n_heads, n_kv_heads, dim);
    float *q_pos = reinterpret_cast<float *>(static_cast<char *>(workspace) + align256(dec_bytes));
    AppendArgs ap{};
    ap.q = q; ap.k = k_new; ap.v = v_new; ap.q_pos = q_pos; ap.kc = k_cache; ap.vc = v_cache;
    ap.n_ctx = n_ctx; ap.H = n_heads; ap.Hkv = n_kv_heads; ap.dim = dim; ap.theta = theta;
    std::vector<int> n_keys(B);
    for (int b0 = 0; b0 < B; b0 += ZT_DEC_MAXB) {
        ap.b_base = b0;
        ap.nb = B - b0 < ZT_DEC_MAXB ? B - b0 : ZT_DEC_MAXB;
        for (int i = 0; i < ap.nb; ++i) ap.pos[i] = pos[b0 + i];
        // One block per 256 tasks of a sequence: (H + Hkv) * dim/2 rotations + Hkv * dim copies.
        const long long tasks = (long long)(n_heads + n_kv_heads) * (dim / 2) + (long long)n_kv_heads * dim;
        const long long blocks = (long long)ap.nb * ((tasks + kThreads - 1) / kThreads);
        if (!grid_ok((unsigned long long)blocks)) return 1;
        if (launch(st, "zt_rope_append", (unsigned)blocks, ap, stream)) return 1;
    }
    for (int b = 0; b < B; ++b) n_keys[b] = pos[b] + 1;
    // Same stream: the attention reads the rows and the rotated queries just written.
    return zt_attn_decode(q_pos, k_cache, v_cache, out, n_keys.data(), B, n_ctx, n_heads, n_kv_heads, dim,
                          workspace, dec_bytes, stream);
}

int zt_rmsnorm_forward(const float *x, const float *w, float *y, int rows, int cols, double eps,
                       hipStream_t stream) {
    if (rows < 0 || cols < 1 || !(eps >= 0.0)) {
        fprintf(stderr, "zt_rmsnorm: %d rows of %d columns with eps %g is not launchable.\n", rows, cols, eps);
        return 1;
    }
    if (rows == 0) return 0;
    if (!x || !w || !y) {
        fprintf(stderr, "zt_rmsnorm: a null tensor pointer is not launchable.\n");
        return 1;
    }
    DeviceState *st = device_state();
    if (!st) {
        fprintf(stderr, "zt_rmsnorm: no usable gfx950 device or code object.\n");
        return 1;
    }
    if (!grid_ok((unsigned long long)rows)) return 1;
    NormArgs a{x, w, y, rows, cols, eps};
    const bool aligned = ((uintptr_t)x % 16 == 0) && ((uintptr_t)w % 16 == 0) && ((uintptr_t)y % 16 == 0);
    const int n4 = cols / 4;
    const char *name = "zt_rmsnorm_any";
    if (cols % 4 == 0 && aligned) {
        if (n4 <= 256) name = "zt_rmsnorm_v1";
        else if (n4 <= 512) name = "zt_rmsnorm_v2";
        else if (n4 <= 1024) name = "zt_rmsnorm_v4";
        else if (n4 <= 2048) name = "zt_rmsnorm_v8";
        else if (n4 <= 4096) name = "zt_rmsnorm_v16";
    }
    return launch(st, name, (unsigned)rows, a, stream);
}

// rows = B * T rows of tensor 1 (heads1 heads) and, when x2 is given, of
// tensor 2 (heads2 heads); row r at position pos + r % T.
static int rope_impl(const char *name, const float *x1, float *y1, const float *x2, float *y2, int B, int T,
                     int heads1, int heads2, int pos, double theta, int head_dim, hipStream_t stream) {
    if (head_dim <= 0 || head_dim % 2 != 0) {
        fprintf(stderr, "zt_rope: head_dim %d is odd or not positive.\n", head_dim);
        return 1;
    }
    if (B < 0 || T < 0 || heads1 < 0 || heads2 < 0 || pos < 0 || (long long)B * T > INT32_MAX) {
        fprintf(stderr, "zt_rope: %d x %d rows of %d + %d heads at position %d is not launchable.\n", B, T, heads1,
                heads2, pos);
        return 1;
    }
    if (!(theta > 0.0)) {
        fprintf(stderr, "zt_rope: theta %g is not usable.\n", theta);
        return 1;
    }
    const long long work = (long long)B * T * (head_dim / 2);
    if (work == 0 || heads1 + heads2 == 0) return 0;
    if (!x1 || !y1 || (heads2 > 0 && (!x2 || !y2))) {
        fprintf(stderr, "zt_rope: a null tensor pointer is not launchable.\n");
        return 1;
    }
    DeviceState *st = device_state();
    if (!st) {
        fprintf(stderr, "zt_rope: no usable gfx950 device or code object.\n");
        return 1;
    }
    RopeArgs a{x1, heads2 > 0 ? x2 : nullptr, y1, heads2 > 0 ? y2 : nullptr, B * T, T, heads1, heads2, pos,
               head_dim, theta};
    long long blocks = (work + kThreads - 1) / kThreads;
    if (blocks > 65536) blocks = 65536;
    return launch(st, name, (unsigned)blocks, a, stream);
}

static int rope_one(const char *name, const float *x, float *y, int rows, int cols, int pos, double theta,
                    int head_dim, hipStream_t stream) {
    if (head_dim <= 0 || head_dim % 2 != 0) {
        fprintf(stderr, "zt_rope: head_dim %d is odd or not positive.\n", head_dim);
        return 1;
    }
    if (rows < 0 || cols < 0 || cols % head_dim != 0) {  // src/rope.zig:30: DimensionMismatch
        fprintf(stderr, "zt_rope: %d rows of %d columns is not a whole number of %d-wide heads.\n", rows, cols,
                head_dim);
        return 1;
    }
    return rope_impl(name, x, y, nullptr, nullptr, 1, rows, cols / head_dim, 0, pos, theta, head_dim, stream);
}

int zt_rope_forward(const float *x, float *y, int rows, int cols, int pos, double theta, int head_dim,
                    hipStream_t stream) {
    return rope_one("zt_rope", x, y, rows, cols, pos, theta, head_dim, stream);
}

int zt_rope_backward(const float *dout, float *din, int rows, int cols, int pos, double theta, int head_dim,
                     hipStream_t stream) {
    return rope_one("zt_rope_bwd", dout, din, rows, cols, pos, theta, head_dim, stream);
}

int zt_rope_qk_forward(const float *q, const float *k, float *q_out, float *k_out, int B, int T, int n_heads,
                       int n_kv_heads, int head_dim, int pos, double theta, hipStream_t stream) {
    return rope_impl("zt_rope", q, q_out, k, k_out, B, T, n_heads, n_kv_heads, pos, theta, head_dim, stream);
}

int zt_rope_qk_backward(const float *dq, const float *dk, float *dq_out, float *dk_out, int B, int T,
                        int n_heads, int n_kv_heads, int head_dim, int pos, double theta, hipStream_t stream) {
    return rope_impl("zt_rope_bwd", dq, dq_out, dk, dk_out, B, T, n_heads, n_kv_heads, pos, theta, head_dim,
                     stream);
}

static int fill_impl(const char *name, float *dst, size_t n, uint64_t seed, double p0, double p1,
                     hipStream_t stream) {
    if (n == 0) return 0;
    if (!dst) {
        fprintf(stderr, "zt_fill: a null pointer is not fillable.\n");
        return 1;
    }
    DeviceState *st = device_state();
    if (!st) {
        fprintf(stderr, "zt_fill: no usable gfx950 device or code object.\n");
        return 1;
    }
    FillArgs a{dst, (unsigned long long)n, (unsigned long long)seed, p0, p1};
    unsigned long long blocks = (n + kThreads - 1) / kThreads;
    if (blocks > 65536) blocks = 65536;
    return launch(st, name, (unsigned)blocks, a, stream);
}

int zt_fill_normal(float *dst, size_t n, uint64_t seed, double mean, double sigma, hipStream_t stream) {
    return fill_impl("zt_fill_normal", dst, n, seed, mean, sigma, stream);
}

int zt_fill_uniform(float *dst, size_t n, uint64_t seed, double lo, double hi, hipStream_t stream) {
    return fill_impl("zt_fill_uniform", dst, n, seed, lo, hi, stream);
}

int zt_attn_plan(int B, int T, int n_heads, int n_kv_heads, int dim, int max_tile, char *fwd, char *dq,
                 char *dkdv, size_t len) {
    if (!fwd || !dq || !dkdv || len < 32 || B < 1 || T < 1 || !zt_attn_dim_ok(dim) || n_heads <= 0 ||
        n_kv_heads <= 0 || n_heads % n_kv_heads != 0 || max_tile < 1)
        return 1;
    DeviceState *st = device_state();
    if (!st) return 1;
    const int dp = pad32(dim);
    int bk = key_tile(Tiled::Forward, dp, max_tile, dim);
    if (fwd_tile_bytes(dp, bk) > st->lds_limit) bk = 32;
    if (T == 1) {  // one query row: the decode kernel
        int G = 0, nw = 0;
        one_row_plan(st, B, n_heads, n_kv_heads, dim, &G, &nw, fwd, len);
    } else {
        const int hw = heads_per_wg(n_heads / n_kv_heads);
        fwd_kernel_name(fwd, len, dim, dp, bk, fwd_waves(hw), fwd_key_split(B, T, n_heads, hw, dp, dim, bk, st->cus));
    }
    BwdArgs a;
    DeviceState *st2 = nullptr;
    unsigned ba = 0, bb = 0, ta = 0, tb = 0;
    char na[64], nb[64];
    // Shape-only planning: the pointers are placeholders that are never
    // dereferenced, aligned as a device allocation is so the choice matches a real call.
    alignas(256) static float dummy[4];
    if (backward_prepare(dummy, dummy, dummy, dummy, dummy, dummy, dummy, dummy, dummy, dummy, B, T,
                         n_heads, n_kv_heads, dim, max_tile, &a, &st2, na, nb, &ba, &bb, &ta, &tb))
        return 1;
    snprintf(dq, len, "%s", na);
    snprintf(dkdv, len, "%s", nb);
    return 0;
}

int zt_attn_plan_train(int B, int T, int n_heads, int n_kv_heads, int dim, char *fwd, char *dq, char *dkdv,
                       size_t len) {
    if (zt_attn_plan(B, T, n_heads, n_kv_heads, dim, 64, fwd, dq, dkdv, len)) return 1;
    DeviceState *st = device_state();
    if (!st) return 1;
    if (T == 1) {  // the training forward keeps lse, so one row still takes the forward kernel
        const int hw = heads_per_wg(n_heads / n_kv_heads), dp = pad32(dim);
        const int bk = key_tile(Tiled::Forward, dp, 64, dim);
        fwd_kernel_name(fwd, len, dim, dp, bk, fwd_waves(hw), fwd_key_split(B, T, n_heads, hw, dp, dim, bk, st->cus));
    }
    const int bt = dqds_tile(B, T, n_heads, dim, st->cus);
    dqds_name(dq, len, bt, dqds_parts(B, T, n_heads, dim, bt, dim % 4 == 0, st->cus));
    const ScoreKernel sk = score_kernel(B, T, dim, n_heads, n_kv_heads, st);
    if (sk == ScoreKernel::RowSplit) {
        snprintf(dkdv, len, "zt_bwd_dkdv_dmars_d%d", pad32(dim));
    } else if (sk == ScoreKernel::Split) {
        const int dp = pad32(dim);
        snprintf(dkdv, len,
                 dp <= 128                        ? "zt_bwd_dkdv8s_d%d_hs2"
                 : dkdv_dsplit(dp, st->lds_limit) ? "zt_bwd_dkdv8sd_d%d_hs2"
                                                  : "zt_bwd_dkdv_dmas_d%d_hs2",
                 dp);
        if (strncmp(fwd, "zt_fwd8p_d", 10) == 0 && dp <= 128) snprintf(fwd, len, "zt_fwd8ps_d%d_k32", dp);
    }
    return 0;
}

int zt_calibrate(const float *src, size_t src_bytes, float *scratch, size_t scratch_bytes, double *mfma_tflops,
                 double *read_gbs, hipStream_t stream) {
    DeviceState *st = require_device();
    if (!st) return 1;
    const unsigned mfma_blocks = (unsigned)st->cus * 4u;  // 4 waves per SIMD
    const unsigned read_blocks = 2048u;
    const size_t need = (size_t)(mfma_blocks > read_blocks ? mfma_blocks : read_blocks) * kThreads * sizeof(float);
    if (!src || !scratch || !mfma_tflops || !read_gbs || scratch_bytes < need || src_bytes < (1u << 20) ||
        (uintptr_t)src % 16 != 0) {
        fprintf(stderr, "zt_calibrate: needs a 16-byte aligned source of at least 1 MiB and %zu bytes of scratch.\n",
                need);
        return 1;
    }
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess) return 1;
    if (hipEventCreate(&e1) != hipSuccess) {
        (void)hipEventDestroy(e0);
        return 1;
    }
    CalArgs a{src, (unsigned long long)(src_bytes / 16), scratch, 20000};
    int rc = 0;
    float best_mfma = 1e30f, best_read = 1e30f;
    for (int rep = 0; rep < 4 && rc == 0; ++rep) {  // the first of each pair warms up; min over the rest
        float ms = 0.f;
        rc |= hipEventRecord(e0, stream) != hipSuccess;
        rc |= launch(st, "zt_cal_mfma", mfma_blocks, a, stream);
        rc |= hipEventRecord(e1, stream) != hipSuccess;
        rc |= hipEventSynchronize(e1) != hipSuccess;
        rc |= hipEventElapsedTime(&ms, e0, e1) != hipSuccess;
        if (rep > 0 && ms < best_mfma) best_mfma = ms;
        rc |= hipEventRecord(e0, stream) != hipSuccess;
        rc |= launch(st, "zt_cal_read", read_blocks, a, stream);
        rc |= hipEventRecord(e1, stream) != hipSuccess;
        rc |= hipEventSynchronize(e1) != hipSuccess;
        rc |= hipEventElapsedTime(&ms, e0, e1) != hipSuccess;
        if (rep > 0 && ms < best_read) best_read = ms;
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (rc) return 1;
    // 2 chains x iters MFMAs of 16 x 16 x 4 x 2 FLOPs per wave, 4 waves per workgroup.
    const double flop = 2.0 * a.iters * 2048.0 * 4.0 * mfma_blocks;
    *mfma_tflops = flop / (best_mfma * 1e-3) / 1e12;
    *read_gbs = (double)a.n4 * 16.0 / (best_read * 1e-3) / 1e9;
    return 0;
}

int zt_calibrate_launch(unsigned blocks, unsigned threads, int launches, double *us_per_launch, hipStream_t stream) {
    DeviceState *st = require_device();
    if (!st) return 1;
    if (!us_per_launch || blocks == 0 || threads == 0 || threads > 1024 || threads % 64 != 0 || launches < 1) {
        fprintf(stderr, "zt_calibrate_launch: %u workgroups of %u threads, %d launches is not a probe.\n", blocks,
                threads, launches);
        return 1;
    }
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess) return 1;
    if (hipEventCreate(&e1) != hipSuccess) {
        (void)hipEventDestroy(e0);
        return 1;
    }
    CalArgs a{};
    int rc = 0;
    float best = 1e30f;
    for (int rep = 0; rep < 4 && rc == 0; ++rep) {  // the first warms up; min over the rest
        float ms = 0.f;
        rc |= hipEventRecord(e0, stream) != hipSuccess;
        for (int i = 0; i < launches && rc == 0; ++i) rc |= launch(st, "zt_cal_empty", blocks, a, stream, threads);
        rc |= hipEventRecord(e1, stream) != hipSuccess;
        rc |= hipEventSynchronize(e1) != hipSuccess;
        rc |= hipEventElapsedTime(&ms, e0, e1) != hipSuccess;
        if (rep > 0 && ms < best) best = ms;
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    if (rc) return 1;
    *us_per_launch = best * 1e3 / launches;
    return 0;
}

// The dense-product kernel for an M x N x K product: slab tile *bt (128, 64
// or 32) with *sk = 0, or split-K tile *bt (16 or 32) with *sk waves.
static void gemm_choose(int M, int N, int K, int n_cus, int *bt_out, int *sk_out) {
    // The largest slab tile whose grid gives every CU a 128-tile, two 64-tiles
    // or 1.5 32-tiles (one 64-tile per CU leaves one wave per SIMD: 1024 x
    // 1024 x 4096 takes 119 us on 64-tiles, 104 us on 32-tiles; 640 x 1024 x
    // 640, 400 32-tiles, 17.4 us against 20.7 us split).  Below that the
    // split-K kernel, with enough waves that each walks at most two 16-deep
    // blocks of K (4 to 16): on 32-tiles when they still give every CU one
    // (512 x 4096 x 512: 39 us, against 49 us on 16-tiles and 60 us on slab
    // 32-tiles), else on 16-tiles (the model's own products, 256 x 512 x 128
    // and the like: 4.1 us, against 6.5 us on 32-tiles and 8.1 us on slabs).
    auto tiles = [&](int t) { return (unsigned long long)((M + t - 1) / t) * (unsigned long long)((N + t - 1) / t); };
    const unsigned long long cus = (unsigned long long)n_cus;
    int bt = 128, sk = 0;
    if (tiles(128) < cus) {
        if (tiles(64) >= 2 * cus) {
            bt = 64;
        } else if (2 * tiles(32) >= 3 * cus) {
            bt = 32;
        } else {
            bt = tiles(32) >= cus ? 32 : 16;
            const int blocks_k = (K + 15) / 16;
            sk = blocks_k <= 8 ? 4 : blocks_k <= 16 ? 8 : 16;
        }
    }
    // A forced slab tile (ZT_GEMM_TILE) takes the slab kernel unless the
    // split is forced too; a forced split (ZT_GEMM_SK > 0) its own tile.
    if (tuned(kTuneGemmTile, 0) != 0 && tuned(kTuneGemmSk, -1) == -1) sk = 0;
    sk = tuned(kTuneGemmSk, sk);
    if (sk) {
        bt = tuned(kTuneGemmSkTile, bt == 32 ? 32 : 16);
    } else {
        bt = tuned(kTuneGemmTile, bt == 16 ? 32 : bt);
    }
    *bt_out = bt;
    *sk_out = sk;
}

// C (+)= op(A) op(B) with the kernel variant `name` (see gemm.hip).
static int gemm_impl(const char *name, const char *what, const float *a, int lda, const float *b, int ldb, float *c,
                     int ldc, int M, int N, int K, int accumulate, hipStream_t stream) {
    if (M < 0 || N < 0 || K < 0) {
        fprintf(stderr, "%s: a %d x %d x %d product is not launchable.\n", what, M, N, K);
        return 1;
    }
    if (M == 0 || N == 0) return 0;  // nothing to write (src/tensor_test.zig:172-183)
    if (!c || (K > 0 && (!a || !b))) {
        fprintf(stderr, "%s: a null tensor pointer is not launchable.\n", what);
        return 1;
    }
    DeviceState *st = device_state();
    if (!st) {
        fprintf(stderr, "%s: no usable gfx950 device or code object.\n", what);
        return 1;
    }
    int bt = 0, sk = 0;
    gemm_choose(M, N, K, st->cus, &bt, &sk);
    auto tiles = [&](int t) { return (unsigned long long)((M + t - 1) / t) * (unsigned long long)((N + t - 1) / t); };
    const unsigned long long blocks = tiles(bt);
    const unsigned threads = sk ? 64u * (unsigned)sk : kThreads;
    if (!grid_ok(blocks, threads)) return 1;
    GemmArgs g{};
    g.a = a; g.b = b; g.c = c;
    g.M = M; g.N = N; g.K = K;
    g.lda = lda; g.ldb = ldb; g.ldc = ldc;
    g.accumulate = accumulate;
    g.vec_a = lda % 4 == 0 && (uintptr_t)a % 16 == 0;
    g.vec_b = ldb % 4 == 0 && (uintptr_t)b % 16 == 0;
    g.vec_c = ldc % 4 == 0 && (uintptr_t)c % 16 == 0;
    char kname[32];
    snprintf(kname, sizeof kname, sk ? "%s_sk%d" : "%s_%d", name, bt);
    return launch(st, kname, (unsigned)blocks, g, stream, threads);
}

int zt_matmul(const float *a, const float *b, float *out, int M, int K, int N, hipStream_t stream) {
    return gemm_impl("zt_gemm_nn", "zt_matmul", a, K, b, N, out, N, M, N, K, 0, stream);
}

int zt_weight_grad(float *w, const float *input, const float *dout, int T, int I, int J, hipStream_t stream) {
    return gemm_impl("zt_gemm_tn", "zt_weight_grad", input, I, dout, J, w, J, I, J, T, 1, stream);
}

int zt_input_grad(float *din, const float *dout, const float *w, int T, int J, int I, hipStream_t stream) {
    return gemm_impl("zt_gemm_nt", "zt_input_grad", dout, J, w, J, din, I, T, I, J, 1, stream);
}

int zt_matmul_plan(int M, int K, int N, char *name, int len) {
    DeviceState *st = device_state();
    if (!st || !name || len < 1 || M < 1 || N < 1 || K < 0) return 1;
    int bt = 0, sk = 0;
    gemm_choose(M, N, K, st->cus, &bt, &sk);
    const int n = sk ? snprintf(name, (size_t)len, "zt_gemm_nn_sk%d", bt) : snprintf(name, (size_t)len, "zt_gemm_nn_%d", bt);
    return n < 0 || n >= len;
}

int zt_attn_set_tuning(const char *name, int value) {
    for (int i = 0; name && i < kTuneCount; ++i) {
        if (strcmp(name, kTuneSpecs[i].name) != 0) continue;
        if (value == -1) {
            g_tune[i].store(0, std::memory_order_relaxed);
            return 0;
        }
        for (int j = 0; j < kTuneSpecs[i].n_allowed; ++j) {
            if (kTuneSpecs[i].allowed[j] == value) {
                g_tune[i].store(value + 1, std::memory_order_relaxed);
                return 0;
            }
        }
        fprintf(stderr, "zt_attn: %d is not a value of the tuning variable %s.\n", value, name);
        return 1;
    }
    fprintf(stderr, "zt_attn: %s is not a tuning variable.\n", name ? name : "(null)");
    return 1;
}

int zt_attn_get_tuning(const char *name) {
    for (int i = 0; name && i < kTuneCount; ++i)
        if (strcmp(name, kTuneSpecs[i].name) == 0) return g_tune[i].load(std::memory_order_relaxed) - 1;
    return -2;
}

const char *zt_attn_version(void) { return "zt_attn gfx950 0.2"; }

size_t zt_attn_lds_limit(void) {
    DeviceState *st = device_state();
    return st ? st->lds_limit : 0;
}

}  // extern "C"
