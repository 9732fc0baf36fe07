// KV-cache decode step: one new query row per sequence against its cached
// keys, split over the key axis (gfx950).
//
// Computes what src/decode.zig:326-392 (attnStep) computes for each sequence
// b: out[b, h] = softmax_s(q[b,h] . k[b,s] / sqrt(d)) v[b,s] over s < n_keys[b],
// with the cache laid out as src/kv_cache.zig:58-63 keeps it ([n_ctx, Hkv*d]
// per sequence).  The reference reaches this through zt_attn_forward with
// T = 1 (src/decode.zig:462); that entry point still works here, this one is
// the bandwidth kernel.
//
// Bound: HBM.  Every K/V byte is read once: a workgroup owns (sequence, kv
// head, key chunk) and serves all G query heads of the group from one read.
// Layout in a wave: LPR = DP/4 lanes cover one cache row with 128-bit loads,
// so one load instruction reads RPI = 64/LPR whole rows (fully coalesced).
// A step is NI such loads of K and of V, and a wave keeps two steps' loads in
// flight (two register buffers, refilled alternately).  For the four-wave
// kernels NI = 4: eight loads per step in one buffer fed from a copy of a
// prefetched one measured C4 652 us and one sequence of 8192 keys 24.6 us;
// two buffers of eight needed 288 registers (one wave per SIMD: 703 us) or
// spilled at 256 (1577 us); two of four: 637 us and 22.5 us.  Partial q.k dots are reduced
// across the LPR lanes with a butterfly reduce-scatter (each exchange halves
// what a lane holds), which leaves every lane with complete scores and costs
// fewer cross-lane moves than one tree per (key, head).  p is broadcast back
// through a small wave-private LDS table; P.V accumulates in registers.
// Per-chunk (max, denominator, accumulator) partials go to a caller-provided
// workspace and zt_dec_combine_* merges them; with one chunk per sequence the
// workgroup writes the output itself and no combine runs.
//
// NW waves per workgroup take a chunk's steps in turn: four when the grid
// fills the device, eight (zt_dec8_*, one or two query heads per workgroup)
// when it cannot -- a single sequence decoded through zt_attn_forward with
// T = 1 has only as many workgroups as (kv head, head sub-group) pairs, and
// then each wave's dependent chain per step (partial dots, butterfly, running
// max, exp, the p broadcast) bounds the rate, so two chains per SIMD instead
// of one nearly halve the time.  Measured on MI355X (one sequence of 8192 keys,
// 32 / 8 heads, d = 128, one query head per workgroup): four waves 237 us,
// eight 143 us; loads two or three steps ahead instead of one gained at most
// 8 % at four waves and nothing at eight, and sixteen waves with half the
// loads per step (to stay within 128 registers) 150 us.
#include <type_traits>

#include "common.h"
#include "args.h"



// Butterfly reduce-scatter over lane masks M, M/2, ..., 1.  On entry v[0..CNT)
// are partial sums; on exit v[0..max(1, CNT/(2M))) are complete sums.
template <int CNT, int M, int V0>
struct Bfly {
    static DEVI void run(float (&v)[V0], int lane) {
        if constexpr (M >= 1) {
            const bool up = (lane & M) != 0;
            if constexpr (CNT > 1) {
#pragma unroll
                for (int j = 0; j < CNT / 2; ++j) {
                    const float send = up ? v[j] : v[j + CNT / 2];
                    const float keep = up ? v[j + CNT / 2] : v[j];
                    v[j] = keep + __shfl_xor(send, M, 64);
                }
                Bfly<CNT / 2, M / 2, V0>::run(v, lane);
            } else {
                v[0] += __shfl_xor(v[0], M, 64);
                Bfly<1, M / 2, V0>::run(v, lane);
            }
        }
    }
};

DEVI float wave_max(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}
DEVI float wave_sum(float v) {
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

template <int DP, int G, int NW, int NI>
__device__ __forceinline__ void decode_body(const DecArgs &a) {
    constexpr int LPR = DP / 4;        // lanes per cache row
    constexpr int RPI = 64 / LPR;      // rows per load instruction
    // NI: load instructions per step (per buffer)
    constexpr int KS = NI * RPI;       // keys per step
    constexpr int V0 = NI * G;         // partial dots per lane
    constexpr int CNT = V0 >= LPR ? V0 / LPR : 1;  // complete scores per lane
    __shared__ float Pl[NW][KS * G];
    __shared__ float Wm[NW][G], Wl[NW][G];
    __shared__ f4 Wacc[NW][G][LPR];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int rg = lane / LPR, sub = lane % LPR;
    const int per_seq = a.n_chunks * a.Hkv * a.n_gsub;
    const int bl = (int)blockIdx.x / per_seq;
    int rem = (int)blockIdx.x % per_seq;
    const int c = rem % a.n_chunks;
    rem /= a.n_chunks;
    const int kvh = rem % a.Hkv, gs = rem / a.Hkv;
    const int b = a.b_base + bl;
    const int nk = a.n_keys[bl];
    const int key0 = c * a.chunk;
    if (key0 >= nk) return;  // workgroup-uniform: nothing of this sequence here
    const int key1 = min(nk, key0 + a.chunk);
    const int group = a.H / a.Hkv;
    const int h0 = kvh * group + gs * G;
    const bool vec4 = (a.dim & 3) == 0;
    const int d0 = 4 * sub;
    const bool dim_ok = d0 < a.dim;
    const size_t kld = (size_t)a.Hkv * a.dim;
    const float *kb = a.kc + (size_t)b * a.n_ctx * kld + (size_t)kvh * a.dim + d0;
    const float *vb = a.vc + (size_t)b * a.n_ctx * kld + (size_t)kvh * a.dim + d0;

    // Cache rows are read exactly once: nontemporal loads keep them from
    // displacing anything in the caches (a streaming read runs at 7.1 TB/s
    // with them on this device, 6.35 TB/s without).
    auto ld4 = [&](const float *p) -> f4 {
        f4 x = zero4();
        if (dim_ok) {
            if (vec4) {
                x = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(p));
            } else {
                const f2 lo = __builtin_nontemporal_load(reinterpret_cast<const f2 *>(p));
                x.x = lo.x; x.y = lo.y;
                if (d0 + 2 < a.dim) {
                    const f2 hi = __builtin_nontemporal_load(reinterpret_cast<const f2 *>(p + 2));
                    x.z = hi.x; x.w = hi.y;
                }
            }
        }
        return x;
    };

    f4 qv[G];
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
        qv[gi] = ld4(a.q + (size_t)b * a.H * a.dim + (size_t)(h0 + gi) * a.dim + d0);
        qv[gi] *= a.scale_log2e;
    }
    f4 acc[G];
    float m[G], ls[G];
#pragma unroll
    for (int gi = 0; gi < G; ++gi) { acc[gi] = zero4(); m[gi] = -INFINITY; ls[gi] = 0.f; }

    const int nsteps = (key1 - key0 + KS - 1) / KS;
    // Two register buffers that the wave's steps alternate between: the loads
    // of a wave's first two steps are both in flight before either is used,
    // and a buffer is refilled (two steps ahead) as soon as its step is done.
    // (Copying a prefetched buffer into a working one made every refill wait
    // for the previous step's data first: one HBM round trip per step, which a
    // single sequence split into short chunks -- two steps per wave -- paid twice.)
    f4 ka[NI], va[NI], kb2[NI], vb2[NI];
    auto load_step = [&](int st, f4 (&kd)[NI], f4 (&vd)[NI]) {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int key = min(key0 + st * KS + i * RPI + rg, nk - 1);  // clamp: stays in the cache
            kd[i] = ld4(kb + (size_t)key * kld);
            vd[i] = ld4(vb + (size_t)key * kld);
        }
    };
    if (w < nsteps) load_step(w, ka, va);
    if (w + NW < nsteps) load_step(w + NW, kb2, vb2);

    // Which (row i, head gi) each of this lane's complete scores belongs to.
    // With fewer partial dots than lanes per row, LPR / V0 lanes hold each complete score.
    constexpr int SHARE = V0 >= LPR ? 1 : LPR / V0;
    int jidx[CNT];
#pragma unroll
    for (int cc = 0; cc < CNT; ++cc) jidx[cc] = (V0 >= LPR) ? sub * CNT + cc : sub / SHARE;
    const bool counted = sub % SHARE == 0;

    auto step = [&](int st, const f4 (&kx)[NI], const f4 (&vx)[NI]) {
        const int kbase = key0 + st * KS;

        float part[V0];
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int gi = 0; gi < G; ++gi) {
                const f4 x = kx[i] * qv[gi];
                part[i * G + gi] = (x.x + x.y) + (x.z + x.w);
            }
        Bfly<V0, LPR / 2, V0>::run(part, lane);

        float sc[CNT];
#pragma unroll
        for (int cc = 0; cc < CNT; ++cc) {
            const int j = jidx[cc];
            const int key = kbase + (j / G) * RPI + rg;
            sc[cc] = key < key1 ? part[cc] : -INFINITY;
        }
        float msafe[G], corr[G];
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            float lm = -INFINITY;
#pragma unroll
            for (int cc = 0; cc < CNT; ++cc)
                if (jidx[cc] % G == gi) lm = fmaxf(lm, sc[cc]);
            const float mnew = fmaxf(m[gi], wave_max(lm));
            msafe[gi] = mnew == -INFINITY ? 0.f : mnew;
            corr[gi] = fast_exp2(m[gi] - msafe[gi]);
            m[gi] = mnew;
            ls[gi] *= corr[gi];
            acc[gi] *= corr[gi];
        }
        float *pl = Pl[w];
#pragma unroll
        for (int cc = 0; cc < CNT; ++cc) {
            const int j = jidx[cc], gi = j % G;
            float ms = msafe[0];
#pragma unroll
            for (int g2 = 1; g2 < G; ++g2) ms = (gi == g2) ? msafe[g2] : ms;
            const float p = fast_exp2(sc[cc] - ms);
            if (counted) {
#pragma unroll
                for (int g2 = 0; g2 < G; ++g2) ls[g2] += (gi == g2) ? p : 0.f;
            }
            pl[((j / G) * RPI + rg) * G + gi] = p;
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const float *pr = pl + (i * RPI + rg) * G;
#pragma unroll
            for (int gi = 0; gi < G; ++gi) acc[gi] += pr[gi] * vx[i];
        }
        __builtin_amdgcn_wave_barrier();
    };

    // The fences keep the compiler from interleaving one step's arithmetic with
    // the other's (which held both steps' temporaries live: 288 registers, one
    // wave per SIMD, against 216 with the steps apart).
    for (int st = w; st < nsteps; st += 2 * NW) {
        step(st, ka, va);
        if (st + 2 * NW < nsteps) load_step(st + 2 * NW, ka, va);
        __builtin_amdgcn_sched_barrier(0);
        if (st + NW < nsteps) {
            step(st + NW, kb2, vb2);
            if (st + 3 * NW < nsteps) load_step(st + 3 * NW, kb2, vb2);
        }
        __builtin_amdgcn_sched_barrier(0);
    }

    // Fold the row groups of this wave, then the NW waves of the workgroup.
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
#pragma unroll
        for (int msk = LPR; msk < 64; msk <<= 1) {
            acc[gi].x += __shfl_xor(acc[gi].x, msk, 64);
            acc[gi].y += __shfl_xor(acc[gi].y, msk, 64);
            acc[gi].z += __shfl_xor(acc[gi].z, msk, 64);
            acc[gi].w += __shfl_xor(acc[gi].w, msk, 64);
        }
        const float lt = wave_sum(ls[gi]);
        if (lane == 0) { Wm[w][gi] = m[gi]; Wl[w][gi] = lt; }
        if (rg == 0) Wacc[w][gi][sub] = acc[gi];
    }
    __syncthreads();
    for (int e = tid; e < G * LPR; e += 64 * NW) {
        const int gi = e / LPR, sb = e % LPR;
        float M = -INFINITY;
        for (int ww = 0; ww < NW; ++ww) M = fmaxf(M, Wm[ww][gi]);
        float L = 0.f;
        f4 A = zero4();
        for (int ww = 0; ww < NW; ++ww) {
            const float f = Wm[ww][gi] == -INFINITY ? 0.f : fast_exp2(Wm[ww][gi] - M);
            L += Wl[ww][gi] * f;
            A += Wacc[ww][gi][sb] * f;
        }
        if (a.n_chunks == 1) {
            // The whole row in one workgroup: the output itself, as the
            // combine would form it (o * (1 / L), the partial's weight being 1).
            const f4 o = A * (1.f / L);
            float *po = a.out + (size_t)b * a.H * a.dim + (size_t)(h0 + gi) * a.dim;
            if (4 * sb < a.dim) {
                if (vec4) {
                    *reinterpret_cast<f4 *>(po + 4 * sb) = o;
                } else {
                    po[4 * sb] = o.x; po[4 * sb + 1] = o.y;
                    if (4 * sb + 2 < a.dim) { po[4 * sb + 2] = o.z; po[4 * sb + 3] = o.w; }
                }
            }
            continue;
        }
        const size_t slot = ((size_t)b * a.H + (h0 + gi)) * a.n_chunks + c;
        float *pa = a.part_acc + slot * a.dim;
        if (4 * sb < a.dim) {
            if (vec4) {
                *reinterpret_cast<f4 *>(pa + 4 * sb) = A;
            } else {
                pa[4 * sb] = A.x; pa[4 * sb + 1] = A.y;
                if (4 * sb + 2 < a.dim) { pa[4 * sb + 2] = A.z; pa[4 * sb + 3] = A.w; }
            }
        }
        if (sb == 0) { a.part_ml[slot * 2] = M; a.part_ml[slot * 2 + 1] = L; }
    }
}

// Block-wide max / sum over the 256 threads of a combine workgroup (red:
// four floats of LDS, reusable: the leading barrier orders a reuse after the
// previous reduction's reads).
DEVI float block_max256(float v, float *red) {
    v = wave_max(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}
DEVI float block_sum256(float v, float *red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// One workgroup per (sequence, query head): merge the chunk partials,
// M = max_c m_c, L = sum_c l_c 2^(m_c - M), out = sum_c acc_c 2^(m_c - M) / L.
// A single sequence split into 64 chunks leaves one short step of work here,
// so what counts is the number of dependent global reads: a thread takes a
// column piece (VW floats: a float4 when the row is, else one float) of
// chunks g, g + NR, ... (NR = 256 / CPT chunk groups, CPT threads covering a
// row), issues the loads of eight chunks' statistics and accumulator pieces
// together, folds them into a running (max, sum, accumulator) of its own, and
// the workgroup merges the threads' triples once: M by a block-wide max, the
// weighted sums through LDS in a fixed order.  Up to 8 NR chunks per sequence
// (the host's default split stays within that) take one round trip to memory.
template <int CPT, int VW>
__device__ __forceinline__ void combine_body(const DecArgs &a) {
    constexpr int NR = 256 / CPT;
    using vec = typename std::conditional<VW == 4, f4, float>::type;
    __shared__ float red[4];
    __shared__ vec part[NR][CPT];
    __shared__ float lpart[NR];
    const int tid = threadIdx.x;
    const int bl = (int)blockIdx.x / a.H, h = (int)blockIdx.x % a.H;
    const int b = a.b_base + bl;
    const int nch = (a.n_keys[bl] + a.chunk - 1) / a.chunk - (ZT_PLANT == 17 ? 1 : 0);
    const size_t slot0 = ((size_t)b * a.H + h) * a.n_chunks;
    const float *ml = a.part_ml + slot0 * 2;
    const int n = tid % CPT, g = tid / CPT;
    const bool col_ok = VW * n < a.dim;
    const float *pa = a.part_acc + slot0 * a.dim + VW * n;
    auto zero = [] { vec z; if constexpr (VW == 4) z = zero4(); else z = 0.f; return z; };
    float mt = -INFINITY, lt = 0.f;
    vec ot = zero();
    for (int c0 = g; c0 < nch; c0 += 8 * NR) {
        float e[8], lv[8];
        vec x[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int c = c0 + j * NR;
            const bool ok = c < nch;
            e[j] = ok ? ml[2 * c] : -INFINITY;
            lv[j] = ok ? ml[2 * c + 1] : 0.f;
            x[j] = (ok && col_ok) ? *reinterpret_cast<const vec *>(pa + (size_t)c * a.dim) : zero();
        }
        float mb = mt;
#pragma unroll
        for (int j = 0; j < 8; ++j) mb = fmaxf(mb, e[j]);
        const float r = mt == -INFINITY ? 0.f : fast_exp2(mt - mb);
        lt *= r;
        ot *= r;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float wj = e[j] == -INFINITY ? 0.f : fast_exp2(e[j] - mb);
            lt += lv[j] * wj;
            ot += x[j] * wj;
        }
        mt = mb;
    }
    const float M = block_max256(mt, red);
    const float f = mt == -INFINITY ? 0.f : fast_exp2(mt - M);
    part[g][n] = ot * f;
    if (n == 0) lpart[g] = lt * f;
    __syncthreads();
    if (g == 0 && col_ok) {
        float L = lpart[0];
        vec sum = part[0][n];
#pragma unroll
        for (int rr = 1; rr < NR; ++rr) {
            L += lpart[rr];
            sum += part[rr][n];
        }
        float *po = a.out + (size_t)b * a.H * a.dim + (size_t)h * a.dim + VW * n;
        *reinterpret_cast<vec *>(po) = sum * (1.f / L);
    }
}

// zt_dec_combine_v<C>: rows of whole float4 (d % 4 == 0), C = the padded
// width / 4 threads per row; zt_dec_combine_s<C>: any even width, one float
// per thread, C threads per row.
#define ZT_DEC_COMBINE(NAME, CPT, VW)                                                              \
    extern "C" __global__ void __launch_bounds__(256) zt_dec_combine_##NAME(DecArgs a) {         \
        combine_body<CPT, VW>(a);                                                                  \
    }
ZT_DEC_COMBINE(v16, 16, 4)
ZT_DEC_COMBINE(v32, 32, 4)
ZT_DEC_COMBINE(v64, 64, 4)
ZT_DEC_COMBINE(s64, 64, 1)
ZT_DEC_COMBINE(s128, 128, 1)
ZT_DEC_COMBINE(s256, 256, 1)

// Two workgroups per CU (two waves per SIMD, at most 256 registers each): the
// grid the host sizes for a full device is two per CU.  Eight heads per
// workgroup do not fit 256 registers without spilling and keep one per CU.
#define ZT_DEC(DP, G)                                                                              \
    extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(G < 8 ? 2 : 1))) \
    zt_dec_d##DP##_g##G(DecArgs a) {                                                               \
        decode_body<DP, G, 4, 4>(a);                                                               \
    }
// Eight waves for one or two query heads per workgroup (more would spill),
// with steps of eight loads: the one-row forward gives a workgroup a whole
// sequence, so it is the step's arithmetic between loads that counts there
// (one C4 sequence of 8192 keys per call: four-load steps 160 us a call,
// eight 144 us; the single-buffer kernel before them 148 us).
#define ZT_DEC8(DP, G)                                                                             \
    extern "C" __global__ void __launch_bounds__(512) zt_dec8_d##DP##_g##G(DecArgs a) {          \
        decode_body<DP, G, 8, 8>(a);                                                               \
    }
#define ZT_DEC_ALL(DP) ZT_DEC(DP, 1) ZT_DEC(DP, 2) ZT_DEC(DP, 4) ZT_DEC(DP, 8) ZT_DEC8(DP, 1) ZT_DEC8(DP, 2)
ZT_DEC_ALL(32)
ZT_DEC_ALL(64)
ZT_DEC_ALL(128)
ZT_DEC_ALL(256)
