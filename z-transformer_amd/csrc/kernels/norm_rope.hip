// RMSNorm, RoPE and seeded fills (gfx950).
//
// zt_rmsnorm_*: src/norm.zig:18-47 on the device, one workgroup per row, one
// HBM read of x (the row stays in registers between the reduction and the
// scale) and one write of y.  The sum of squares accumulates in f64 (each f32
// square is exact in f64, so only the summation order differs from the
// reference's sequential loop), rms = f32(sqrt(sum/d + eps)) exactly as
// norm.zig:41 narrows it, then y = x / rms * w with an IEEE f32 divide and an
// f32 multiply (norm.zig:44).  Bound: HBM (8 bytes per element + the gain).
//
// zt_rope / zt_rope_bwd: src/rope.zig:21-55 and its transpose
// src/autograd.zig:851-872 (half-split pairs i <-> i + d/2, f64 angle
// t / theta^(2i/d), f64 products, one narrowing).  The angle depends on
// (position, i) only, so one thread computes pow, cos and sin once and applies
// them to pair i of every head of the row -- of q and k together when both are
// given -- which keeps the f64 transcendentals off the critical path and the
// kernel near HBM speed.  Products and sums are kept as separate roundings
// (no fused multiply-add), as the reference computes them.
//
// zt_fill_normal / zt_fill_uniform: counter-based splitmix64 -> Box-Muller,
// element i from counters 2i and 2i+1, so a buffer of any size is filled in
// parallel and reproducibly.
#include "common.h"
#include "args.h"


DEVI double wave_sum_d(double v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// Block-wide f64 sum over NWV waves (a workgroup of 64 * NWV threads): each
// wave's sum goes to red[w], and the NWV of them are added as a pairwise tree
// (for four waves (r0 + r1) + (r2 + r3)).
template <int NWV>
DEVI double block_sum_d(double v, double (&red)[NWV]) {
    static_assert(NWV >= 1 && (NWV & (NWV - 1)) == 0, "the wave count must be a power of two");
    v = wave_sum_d(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    double t[NWV];
#pragma unroll
    for (int i = 0; i < NWV; ++i) t[i] = red[i];
#pragma unroll
    for (int n = NWV; n > 1; n >>= 1)
#pragma unroll
        for (int i = 0; i < n / 2; ++i) t[i] = t[2 * i] + t[2 * i + 1];
    return t[0];
}

// cols % 4 == 0: each of the 256 threads keeps NV float4 of the row (cols <= 1024 * NV).
// (A 1024-thread workgroup holding one float4 per thread measured slower at
// [64, 4096] on MI355X: 3.35 us against 3.20 us per kernel in a replayed graph,
// where an empty kernel of the same grid costs 2.39 us per launch.)
template <int NV, int NTH = 256>
__device__ __forceinline__ void rms_vec(const NormArgs &a) {
    __shared__ double red[NTH / 64];
    const int r = blockIdx.x;
    const float *xr = a.x + (size_t)r * a.cols;
    float *yr = a.y + (size_t)r * a.cols;
    const int n4 = a.cols >> 2;
    f4 xv[NV];
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = threadIdx.x + NTH * i;
        // x is read once and y written once: nontemporal, so neither displaces
        // the gain row every workgroup rereads.
        xv[i] = c < n4 ? __builtin_nontemporal_load(reinterpret_cast<const f4 *>(xr) + c) : zero4();
        if constexpr (ZT_PLANT == 22) {
            ss += (double)xv[i].x + (double)xv[i].y + (double)xv[i].z + (double)xv[i].w;
        } else {
            ss += (double)xv[i].x * (double)xv[i].x;
            ss += (double)xv[i].y * (double)xv[i].y;
            ss += (double)xv[i].z * (double)xv[i].z;
            ss += (double)xv[i].w * (double)xv[i].w;
        }
    }
    const double tot = block_sum_d(ss, red);
    const float rms = (float)sqrt(tot / (double)a.cols + a.eps);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = threadIdx.x + NTH * i;
        if (c < n4) {
            f4 wv = reinterpret_cast<const f4 *>(ZT_PLANT == 23 ? xr : a.w)[c];
            if (ZT_PLANT == 21 && c == 0) wv.x += 1e-3f;
            f4 yv;
            yv.x = xv[i].x / rms * wv.x;
            yv.y = xv[i].y / rms * wv.y;
            yv.z = xv[i].z / rms * wv.z;
            yv.w = xv[i].w / rms * wv.w;
            __builtin_nontemporal_store(yv, reinterpret_cast<f4 *>(yr) + c);
        }
    }
}

// Any cols: scalar elements, row re-read for the scale pass (L2-resident).
__device__ __forceinline__ void rms_any(const NormArgs &a) {
    __shared__ double red[4];
    const int r = blockIdx.x;
    const float *xr = a.x + (size_t)r * a.cols;
    float *yr = a.y + (size_t)r * a.cols;
    double ss = 0.0;
    for (int c = threadIdx.x; c < a.cols; c += 256) ss += (double)xr[c] * (double)xr[c];
    const double tot = block_sum_d(ss, red);
    const float rms = (float)sqrt(tot / (double)a.cols + a.eps);
    for (int c = threadIdx.x; c < a.cols; c += 256) yr[c] = xr[c] / rms * a.w[c];
}

#define ZT_RMS(NV)                                                                                 \
    extern "C" __global__ void __launch_bounds__(256) zt_rmsnorm_v##NV(NormArgs a) { rms_vec<NV>(a); }
ZT_RMS(1)
ZT_RMS(2)
ZT_RMS(4)
ZT_RMS(8)
ZT_RMS(16)
extern "C" __global__ void __launch_bounds__(256) zt_rmsnorm_any(NormArgs a) { rms_any(a); }


#pragma clang fp contract(off)

// cos and sin of the RoPE angle of pair i at position t (src/rope.zig:40-43).
DEVI void rope_angle(double t, int i, int head_dim, double theta, double *c, double *s) {
    const double exponent = (double)(2 * i) / (double)head_dim;
    const double angle = t / pow(theta, exponent);
    *c = cos(angle);
    *s = sin(angle);
}

// Rotates the pair (lo, hi): forward (rope.zig:47-48) lo c - hi s, hi c + lo s;
// backward, the transpose (autograd.zig:867-868), lo c + hi s, hi c - lo s.
template <bool BWD>
DEVI void rope_rotate(double c, double s, const float *x, float *y, int half) {
    const double lo = (double)x[0], hi = (double)x[half];
    const double lc = lo * c, hs = hi * s, hc = hi * c, ls = lo * s;
    y[0] = (float)(BWD ? lc + hs : lc - hs);
    y[half] = (float)(BWD ? hc - ls : hc + ls);
}

template <bool BWD>
DEVI void rope_rows(const RopeArgs &a) {
    const int half = a.head_dim / 2;
    const size_t ld1 = (size_t)a.heads1 * a.head_dim, ld2 = (size_t)a.heads2 * a.head_dim;
    const long long total = (long long)a.rows * half;
    for (long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (long long)gridDim.x * blockDim.x) {
        const int i = (int)(e % half);
        const int r = (int)(e / half);
        double c, s;
        rope_angle((double)(a.pos + r % a.seq_len), i, a.head_dim, a.theta, &c, &s);
        const float *x1 = a.x1 + (size_t)r * ld1 + i;
        float *y1 = a.y1 + (size_t)r * ld1 + i;
        for (int h = 0; h < a.heads1; ++h)
            rope_rotate<BWD>(c, s, x1 + (size_t)h * a.head_dim, y1 + (size_t)h * a.head_dim, half);
        const float *x2 = a.x2 + (size_t)r * ld2 + i;
        float *y2 = a.y2 + (size_t)r * ld2 + i;
        for (int h = 0; h < a.heads2; ++h)
            rope_rotate<BWD>(c, s, x2 + (size_t)h * a.head_dim, y2 + (size_t)h * a.head_dim, half);
    }
}

extern "C" __global__ void __launch_bounds__(256) zt_rope(RopeArgs a) { rope_rows<false>(a); }
extern "C" __global__ void __launch_bounds__(256) zt_rope_bwd(RopeArgs a) { rope_rows<true>(a); }

// Decode-step cache update (src/decode.zig:244-259: rope.forward on q and k
// at pos, cache append).  A sequence's work -- (H + Hkv) * d/2 pair rotations
// and Hkv * d copies of the new v into cache row pos[b] -- is cut into
// 256-task blocks, blockIdx.x = sequence * blocks_per_seq + piece.  Each block
// first tabulates cos / sin of its sequence's d/2 angles in LDS (one f64 pow,
// cos, sin per pair), then every thread does one task, so the launch is wide
// and a thread's loads do not queue behind one another.
extern "C" __global__ void __launch_bounds__(256) zt_rope_append(AppendArgs a) {
    __shared__ double tab_c[ZT_MAX_DIM / 2], tab_s[ZT_MAX_DIM / 2];
    const int half = a.dim / 2;
    const int n_rot = (a.H + a.Hkv) * half;
    const int tasks = n_rot + a.Hkv * a.dim;
    const int per_seq = (tasks + 255) / 256;
    const int bl = blockIdx.x / per_seq, piece = blockIdx.x % per_seq;
    if (bl >= a.nb) return;  // block-uniform
    const int b = a.b_base + bl;
    const int pos = a.pos[bl];
    for (int i = threadIdx.x; i < half; i += blockDim.x) rope_angle((double)pos, i, a.dim, a.theta, &tab_c[i], &tab_s[i]);
    __syncthreads();
    const int j = piece * 256 + threadIdx.x;
    if (j >= tasks) return;
    const size_t qld = (size_t)a.H * a.dim, kld = (size_t)a.Hkv * a.dim;
    if (j < n_rot) {
        const int h = j / half, i = j % half;
        if (h < a.H) {
            const size_t o = (size_t)b * qld + (size_t)h * a.dim + i;
            rope_rotate<false>(tab_c[i], tab_s[i], a.q + o, a.q_pos + o, half);
        } else {
            const size_t col = (size_t)(h - a.H) * a.dim + i;
            rope_rotate<false>(tab_c[i], tab_s[i], a.k + (size_t)b * kld + col,
                               a.kc + ((size_t)b * a.n_ctx + pos) * kld + col, half);
        }
    } else {
        const int c = j - n_rot;
        a.vc[((size_t)b * a.n_ctx + pos) * kld + c] = a.v[(size_t)b * kld + c];
    }
}

DEVI unsigned long long splitmix64(unsigned long long seed, unsigned long long ctr) {
    unsigned long long z = seed + (ctr + 1ull) * 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
DEVI double unit53(unsigned long long x) { return (double)(x >> 11) * 0x1.0p-53; }

extern "C" __global__ void __launch_bounds__(256) zt_fill_normal(FillArgs a) {
    const double two_pi = 6.283185307179586476925286766559;
    for (unsigned long long i = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x; i < a.n;
         i += (unsigned long long)gridDim.x * blockDim.x) {
        const double u1 = 1.0 - unit53(splitmix64(a.seed, 2 * i));
        const double u2 = unit53(splitmix64(a.seed, 2 * i + 1));
        a.dst[i] = (float)(a.p0 + a.p1 * (sqrt(-2.0 * log(u1)) * cos(two_pi * u2)));
    }
}

extern "C" __global__ void __launch_bounds__(256) zt_fill_uniform(FillArgs a) {
    for (unsigned long long i = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x; i < a.n;
         i += (unsigned long long)gridDim.x * blockDim.x)
        a.dst[i] = (float)(a.p0 + (a.p1 - a.p0) * unit53(splitmix64(a.seed, i)));
}
