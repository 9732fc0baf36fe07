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
// zt_rope: src/rope.zig:21-55 (half-split pairs i <-> i + d/2, f64 angle
// t / theta^(2i/d), f64 multiply-adds, one narrowing).  Used to prepare
// RoPE-rotated inputs.
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

// Block-wide f64 sum over 256 threads.
DEVI double block_sum_d(double v, double *red) {
    v = wave_sum_d(v);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// cols % 4 == 0: each thread keeps NV float4 of the row (cols <= 1024 * NV).
template <int NV>
__device__ __forceinline__ void rms_vec(const NormArgs &a) {
    __shared__ double red[4];
    const int r = blockIdx.x;
    const float *xr = a.x + (size_t)r * a.cols;
    float *yr = a.y + (size_t)r * a.cols;
    const int n4 = a.cols >> 2;
    f4 xv[NV];
    double ss = 0.0;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = threadIdx.x + 256 * i;
        xv[i] = c < n4 ? reinterpret_cast<const f4 *>(xr)[c] : zero4();
        ss += (double)xv[i].x * (double)xv[i].x;
        ss += (double)xv[i].y * (double)xv[i].y;
        ss += (double)xv[i].z * (double)xv[i].z;
        ss += (double)xv[i].w * (double)xv[i].w;
    }
    const double tot = block_sum_d(ss, red);
    const float rms = (float)sqrt(tot / (double)a.cols + a.eps);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = threadIdx.x + 256 * i;
        if (c < n4) {
            const f4 wv = reinterpret_cast<const f4 *>(a.w)[c];
            f4 yv;
            yv.x = xv[i].x / rms * wv.x;
            yv.y = xv[i].y / rms * wv.y;
            yv.z = xv[i].z / rms * wv.z;
            yv.w = xv[i].w / rms * wv.w;
            reinterpret_cast<f4 *>(yr)[c] = yv;
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


// Transposed rotation, src/autograd.zig:851-872: (lo c + hi s, hi c - lo s).
extern "C" __global__ void __launch_bounds__(256) zt_rope_bwd(RopeArgs a) {
    const int half = a.head_dim / 2;
    const int heads = a.cols / a.head_dim;
    const long long total = (long long)a.rows * heads * half;
    for (long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (long long)gridDim.x * blockDim.x) {
        const int i = (int)(e % half);
        const long long rh = e / half;
        const int h = (int)(rh % heads);
        const int r = (int)(rh / heads);
        const double t = (double)(a.pos + r);
        const double exponent = (double)(2 * i) / (double)a.head_dim;
        const double angle = t / pow(a.theta, exponent);
        const double c = cos(angle), s = sin(angle);
        const size_t base = (size_t)r * a.cols + (size_t)h * a.head_dim;
        const double lo = (double)a.x[base + i], hi = (double)a.x[base + i + half];
        a.y[base + i] = (float)(lo * c + hi * s);
        a.y[base + i + half] = (float)(hi * c - lo * s);
    }
}

extern "C" __global__ void __launch_bounds__(256) zt_rope(RopeArgs a) {
    const int half = a.head_dim / 2;
    const int heads = a.cols / a.head_dim;
    const long long total = (long long)a.rows * heads * half;
    for (long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (long long)gridDim.x * blockDim.x) {
        const int i = (int)(e % half);
        const long long rh = e / half;
        const int h = (int)(rh % heads);
        const int r = (int)(rh / heads);
        const double t = (double)(a.pos + r);
        const double exponent = (double)(2 * i) / (double)a.head_dim;
        const double angle = t / pow(a.theta, exponent);
        const double c = cos(angle), s = sin(angle);
        const size_t base = (size_t)r * a.cols + (size_t)h * a.head_dim;
        const double lo = (double)a.x[base + i], hi = (double)a.x[base + i + half];
        a.y[base + i] = (float)(lo * c - hi * s);
        a.y[base + i + half] = (float)(hi * c + lo * s);
    }
}


// RoPE rotation of the pair (lo, hi) = (x[i], x[i + d/2]) at position t, as
// src/rope.zig:37-50: f64 angle t / theta^(2i/d), f64 multiply-adds.
DEVI void rope_pair(double t, int i, int head_dim, double theta, float lo_in, float hi_in, float *lo_out,
                    float *hi_out) {
    const double exponent = (double)(2 * i) / (double)head_dim;
    const double angle = t / pow(theta, exponent);
    const double c = cos(angle), s = sin(angle);
    const double lo = (double)lo_in, hi = (double)hi_in;
    *lo_out = (float)(lo * c - hi * s);
    *hi_out = (float)(hi * c + lo * s);
}

// Decode-step cache update, one thread per element task: rotated q pairs,
// rotated k pairs written to cache row pos[b], v elements copied to row pos[b]
// (src/decode.zig:244-259: rope.forward on q and k at pos, cache append).
extern "C" __global__ void __launch_bounds__(256) zt_rope_append(AppendArgs a) {
    const int half = a.dim / 2;
    const long long nq = (long long)a.nb * a.H * half;
    const long long nk = (long long)a.nb * a.Hkv * half;
    const long long nv = (long long)a.nb * a.Hkv * a.dim;
    const size_t qld = (size_t)a.H * a.dim, kld = (size_t)a.Hkv * a.dim;
    for (long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x; e < nq + nk + nv;
         e += (long long)gridDim.x * blockDim.x) {
        if (e < nq) {
            const int i = (int)(e % half);
            const long long bh = e / half;
            const int h = (int)(bh % a.H), bl = (int)(bh / a.H);
            const size_t o = (size_t)(a.b_base + bl) * qld + (size_t)h * a.dim;
            rope_pair((double)a.pos[bl], i, a.dim, a.theta, a.q[o + i], a.q[o + i + half], &a.q_pos[o + i],
                      &a.q_pos[o + i + half]);
        } else if (e < nq + nk) {
            const long long f = e - nq;
            const int i = (int)(f % half);
            const long long bh = f / half;
            const int h = (int)(bh % a.Hkv), bl = (int)(bh / a.Hkv);
            const int b = a.b_base + bl;
            const size_t src = (size_t)b * kld + (size_t)h * a.dim;
            const size_t dst = ((size_t)b * a.n_ctx + a.pos[bl]) * kld + (size_t)h * a.dim;
            rope_pair((double)a.pos[bl], i, a.dim, a.theta, a.k[src + i], a.k[src + i + half], &a.kc[dst + i],
                      &a.kc[dst + i + half]);
        } else {
            const long long f = e - nq - nk;
            const int c = (int)(f % kld);
            const int bl = (int)(f / kld);
            const int b = a.b_base + bl;
            a.vc[((size_t)b * a.n_ctx + a.pos[bl]) * kld + c] = a.v[(size_t)b * kld + c];
        }
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
