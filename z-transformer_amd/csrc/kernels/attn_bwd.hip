// Fused causal grouped-query attention, backward, f32 on FP32 MFMA (gfx950).
//
// Two kernels on one stream, no atomics, so every run is bit-reproducible --
// the determinism argument of src/cuda/attn_kernels.cu:538-543 kept, with a
// different schedule:
//
// Kernel A (zt_bwd_dq_*), Q-outer.  Same workgroup shape as the forward: 4
// waves = HW query heads of one kv group x (4 / HW) blocks of 16 rows, K/V
// tiles staged in LDS once per kv group.  Per key tile it forms
// S^T = K Q^T and dP^T = V dO^T on MFMA, keeps the online softmax, and
// accumulates a0 = sum_s p~ k_s and a1 = sum_s p~ dp_s k_s, so that at the end
//     delta = sum p~ dp / l,   dq = scale (a1 - delta a0) / l
// -- the identity src/cuda/attn_kernels.cu:508-517 uses (dq = sum_s
// p (dp - delta) k scale, autograd.zig:799-820).  It writes the per-row
// row_max (natural units), row_den and row_del, the scratch contract of
// attn_kernels.cu:520-532.
//
// Kernel B (zt_bwd_dkdv_*), KV-outer.  A workgroup owns 16*KW keys of one kv
// group: wave (kb, hs) owns 16 keys and every HS-th query head of the group.
// K and V stay in registers; Q and dO rows are staged in LDS 16 rows at a
// time for the suffix t >= s.  With the row statistics from kernel A:
//     p = exp(S - row_max) / row_den,  dS = p (dP - row_del)
//     dV^T += dO^T P,   dK^T += Q^T dS      (MFMA, P and dS register-resident)
// The HS head-split partials are summed in LDS in a fixed order at the end.
// dv carries no scale, dk carries 1/sqrt(d) (autograd.zig:829-836).
#include "common.h"
#include "args.h"


// The K and V tiles of the dq kernels: one allocation per (DP, BK), shared by
// a kernel's instantiations for aligned and unaligned rows.
template <int DP, int BK>
__device__ __forceinline__ float *dq_kv_tiles() {
    __shared__ float kv[2 * BK * (DP + 4)];
    return kv;
}

template <int DP, int BK, int NW, bool PF = false, bool VEC = false>
__device__ __forceinline__ void bwd_dq_tile(const BwdArgs &a, const int tile) {
    constexpr int LW = DP + 4, DQ = DP / 4, NT = DP / 16, NJ = BK / 16;
    float *const Ks = dq_kv_tiles<DP, BK>(), *const Vs = Ks + BK * LW;

    const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, grp = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // in a scalar register: wave-uniform branches stay scalar
    const int RB = NW / a.HW;  // 16-row blocks per head in this workgroup
    const int per_tile = a.n_head_blocks * a.B;
    const int rem = (int)blockIdx.x % per_tile;
    const int hb = rem % a.n_head_blocks, b = rem / a.n_head_blocks;
    const int group = a.H / a.Hkv;
    const int h = hb * a.HW + (w % a.HW);
    const int kvh = ZT_PLANT == 12 ? 0 : h / group;
    const int wg_row0 = tile * 16 * RB;
    const int row0 = wg_row0 + 16 * (w / a.HW);
    const bool vec4 = (a.dim & 3) == 0;
    const size_t qld = (size_t)a.H * a.dim, kld = (size_t)a.Hkv * a.dim;
    const size_t qoff = (size_t)b * a.T * qld + (size_t)h * a.dim;
    const float *kb = a.k + (size_t)b * a.T * kld + (size_t)kvh * a.dim;
    const float *vb = a.v + (size_t)b * a.T * kld + (size_t)kvh * a.dim;

    const int my_row = row0 + l16;
    const bool row_ok = my_row < a.T;
    float qr[DQ], dor[DQ];
    load_row_seg<DQ>(qr, a.q + qoff + (size_t)my_row * qld, grp * DQ, a.dim, vec4, row_ok,
                     ZT_PLANT == 14 ? kLog2e : a.scale_log2e);
    load_row_seg<DQ>(dor, a.dout + qoff + (size_t)my_row * qld, grp * DQ, a.dim, vec4, row_ok, 1.f);

    f4 a0[NT], a1[NT];
#pragma unroll
    for (int i = 0; i < NT; ++i) { a0[i] = zero4(); a1[i] = zero4(); }
    float m = -INFINITY, mx = -INFINITY, lsum = 0.f, dlsum = 0.f;
    const int kend_wg = min(a.T, wg_row0 + 16 * RB);
    const int kend_w = row0 < a.T ? min(a.T, row0 + 16) : 0;

    // Register prefetch (PF) of the next K/V tile, as in the forward.
    constexpr int NTH = 64 * NW, CPR = DP / 4;
    constexpr int NPF = PF ? 2 * BK * CPR / NTH : 1;
    static_assert(!PF || (2 * BK * CPR) % NTH == 0, "prefetch split");
    f4 pf[NPF];
    // VEC (dim % 4 == 0, 16-byte aligned rows): every load unconditional and
    // in bounds, so the pieces go out between the score products -- keys past
    // T load key T - 1 (masked, P = 0) and columns past dim the row's last
    // chunk (met by Q's and dO's zero columns, or landing in dq columns never
    // stored).  Otherwise guarded loads, all at the top of the tile.
    // VEC: a thread's byte offsets within a tile's rows are fixed for the
    // kernel (rows tid / CPR + j RPN, its column): a piece is one load from the
    // tile's base plus the offset clamped (one min) to key T - 1, as in the
    // forward (d <= 128: C3 dq kernels 2.045 -> 2.035 ms; at d = 256 the
    // statistics-building one spills more and loses, 1.28 -> 1.32 ms).
    constexpr int RPN = NTH / CPR;
    constexpr int NOFF = DP <= 128 && (BK * CPR) % NTH == 0 && BK % RPN == 0 ? BK / RPN : 1;
    unsigned voff[NOFF];
    const unsigned coff = (unsigned)min((tid % CPR) * 4, a.dim - 4) * 4u;
#pragma unroll
    for (int j = 0; j < NOFF; ++j) voff[j] = (unsigned)((tid / CPR + j * RPN) * (int)kld) * 4u + coff;
    auto fetch_piece = [&](int n, int k0) {
        const int e = tid + n * NTH;
        const int arr = e / (BK * CPR), r = (e / CPR) % BK, c = (e % CPR) * 4;
        if constexpr (VEC && NOFF > 1) {
            // Key T - 1, counted within the tile (no 32-bit overflow however long T is).
            const unsigned last = (unsigned)(min(a.T - 1 - k0, BK - 1) * (int)kld) * 4u + coff;
            const unsigned off = min(voff[(n * RPN % BK) / RPN], last);
            pf[n] = *reinterpret_cast<const f4 *>(reinterpret_cast<const char *>((arr ? vb : kb) + (size_t)k0 * kld) + off);
        } else if constexpr (VEC) {
            pf[n] = *reinterpret_cast<const f4 *>((arr ? vb : kb) + (size_t)k0 * kld +
                                                  (min(r, a.T - 1 - k0) * (int)kld + min(c, a.dim - 4)));
        } else {
            const int key = k0 + r;
            const float *src = (arr ? vb : kb) + (size_t)key * kld + c;
            f4 x = zero4();
            if (key < a.T && c < a.dim) {
                if (vec4) {
                    x = *reinterpret_cast<const f4 *>(src);
                } else {
                    const f2 lo = *reinterpret_cast<const f2 *>(src);
                    x.x = lo.x; x.y = lo.y;
                    if (c + 2 < a.dim) {
                        const f2 hi = *reinterpret_cast<const f2 *>(src + 2);
                        x.z = hi.x; x.w = hi.y;
                    }
                }
            }
            pf[n] = x;
        }
    };
    auto fetch = [&](int k0) {
#pragma unroll
        for (int n = 0; n < NPF; ++n) fetch_piece(n, k0);
    };
    // Pieces of group i of NI between the score products (VEC, up to d = 192).
    auto fetch_group = [&](int i, int ni, int k0) {
#pragma unroll
        for (int n = i * NPF / ni; n < (i + 1) * NPF / ni; ++n) fetch_piece(n, k0);
    };
    if constexpr (PF) fetch(0);

    // Interleaved prefetch: VEC kernels whose score loop runs k-step outer.
    constexpr bool ILV = PF && VEC && DP <= 192;
    for (int k0 = 0; k0 < kend_wg; k0 += BK) {
        __syncthreads();
        const int kn = k0 + BK < kend_wg ? k0 + BK : k0;  // the last tile fetches itself again, unused
        if constexpr (PF) {
#pragma unroll
            for (int n = 0; n < NPF; ++n) {
                const int e = tid + n * NTH;
                const int arr = e / (BK * CPR), r = (e / CPR) % BK, c = (e % CPR) * 4;
                *reinterpret_cast<f4 *>((arr ? Vs : Ks) + r * LW + c) = pf[n];
            }
            __syncthreads();
            if constexpr (!ILV) {
                if (k0 + BK < kend_wg) fetch(k0 + BK);
            }
        } else {
            const int nvalid = min(BK, a.T - k0);
            stage_rows<DP, LW, NTH>(Ks, kb + (size_t)k0 * kld, kld, BK, nvalid, a.dim, vec4, tid);
            stage_rows<DP, LW, NTH>(Vs, vb + (size_t)k0 * kld, kld, BK, nvalid, a.dim, vec4, tid);
            __syncthreads();
        }
        if (k0 >= kend_w) {  // wave-uniform: nothing here is visible to this wave
            if constexpr (ILV) fetch(kn);
            continue;
        }

        // S^T and dP^T for every 16-key sub-block.  Up to d = 192 the 2 * NJ
        // independent accumulation chains are interleaved so consecutive MFMAs
        // do not wait on each other; wider heads keep one sub-block at a time
        // (interleaving them would spill).  Wholly invisible sub-blocks are
        // computed and then masked.
        f4 s[NJ], dp[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) { s[j] = zero4(); dp[j] = zero4(); }
        const float *krow = Ks + l16 * LW + grp * DQ;
        const float *vrow = Vs + l16 * LW + grp * DQ;
        auto score_step = [&](int j, int kk) {
            const f4 kx = *reinterpret_cast<const f4 *>(krow + 16 * j * LW + kk);
            const f4 vx = *reinterpret_cast<const f4 *>(vrow + 16 * j * LW + kk);
            s[j] = mfma16(kx.x, qr[kk + 0], s[j]);
            dp[j] = mfma16(vx.x, dor[kk + 0], dp[j]);
            s[j] = mfma16(kx.y, qr[kk + 1], s[j]);
            dp[j] = mfma16(vx.y, dor[kk + 1], dp[j]);
            s[j] = mfma16(kx.z, qr[kk + 2], s[j]);
            dp[j] = mfma16(vx.z, dor[kk + 2], dp[j]);
            s[j] = mfma16(kx.w, qr[kk + 3], s[j]);
            dp[j] = mfma16(vx.w, dor[kk + 3], dp[j]);
        };
        if constexpr (DP <= 192) {
#pragma unroll
            for (int kk = 0; kk < DQ; kk += 4) {
#pragma unroll
                for (int j = 0; j < NJ; ++j) score_step(j, kk);
                if constexpr (ILV) fetch_group(kk / 4, DQ / 4, kn);
            }
        } else {
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int kk = 0; kk < DQ; kk += 4) score_step(j, kk);
        }
        if (k0 + BK - 1 > row0 || k0 + BK > a.T) {  // wave-uniform: a key past a row or past T
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int key = k0 + 16 * j + 4 * grp + r;
                    if ((ZT_PLANT != 11 && key > my_row) || key >= a.T) s[j][r] = -INFINITY;
                }
            }
        }
        float mt = -INFINITY;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
            mt = fmaxf(mt, fmaxf(fmaxf(s[j][0], s[j][1]), fmaxf(s[j][2], s[j][3])));
        mt = max4grp(mt);
        mx = fmaxf(mx, mt);
        // Lazy rescaling, as in the forward: the exponent base m of a row moves
        // only when the row meets a tile maximum more than 8 (log2 units) above
        // it, so the 2 NT accumulators need rescaling only then (the reference
        // entry point's backward: C3 4.27 -> 4.23 ms, C5 2.63 -> 2.54 ms, with a
        // 9-VGPR spill at d = 128).  The true maximum mx is kept beside it for
        // the row statistics.
        if (mt > m + 8.f) {
            const float mnew = fmaxf(m, mt);
            const float corr = fast_exp2(m - mnew);
            m = mnew;
            lsum *= corr;
            dlsum *= corr;
#pragma unroll
            for (int i = 0; i < NT; ++i) { a0[i] *= corr; a1[i] *= corr; }
        }
        float ps = 0.f, pds = 0.f;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float p = fast_exp2(s[j][r] - m);
                s[j][r] = p;
                dp[j][r] *= p;  // p~ dp
                ps += p;
                pds += dp[j][r];
            }
        lsum += ps;
        dlsum += pds;

#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            if (k0 + 16 * j >= kend_w) continue;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const float pv = s[j][kk], pd = dp[j][kk];
                float kx[NT];  // K^T rows, row-owner layout: K[key][l16 * NT + i]
                lds_run<NT>(kx, Ks + (16 * j + 4 * grp + kk) * LW, l16);
#pragma unroll
                for (int i = 0; i < NT; ++i) {
                    a0[i] = mfma16(kx[i], pv, a0[i]);
                    a1[i] = mfma16(kx[i], pd, a1[i]);
                }
            }
        }
    }

    const float l = sum4grp(lsum);
    const float delta = sum4grp(dlsum) / l;
    const float f = (ZT_PLANT == 14 ? 1.f : a.scale) / l;
    if (row_ok) {
        float *dqrow = a.dq + qoff + (size_t)my_row * qld;
#pragma unroll
        for (int i = 0; i < NT; ++i) a1[i] = ZT_PLANT == 13 ? a0[i] : a1[i] - delta * a0[i];
#pragma unroll
        for (int r = 0; r < 4; ++r) store_run<NT>(dqrow, 4 * grp + r, a.dim, vec4, a1, r, f);
        if (grp == 0) {
            const size_t o = ((size_t)b * a.T + my_row) * a.H + h;
            // The statistics against the row's true maximum (natural units), as
            // the reference's scratch contract has them: l was summed against m.
            a.row_max[o] = mx * 0.69314718055994531f;
            a.row_den[o] = l * fast_exp2(m - mx);
            a.row_del[o] = delta;
        }
    }
}

// dq from saved statistics (training path: the forward wrote lse and o).
// Per row: delta = sum_d o * dO (written to row_del for the dk/dv kernel);
// per key tile: S^T = K Q^T, P = exp2(S - lse2) (no running max, no
// rescaling), dP^T = V dO^T, dS = P (dP - delta), dq^T += K^T dS^T -- three
// matmul units instead of the four the statistics-building kernel needs.
// K/V tiles are register-prefetched as in bwd_dq_body.
template <int DP, int BK, int NW, bool VEC = false>
__device__ __forceinline__ void bwd_dq_lse_tile(const BwdArgs &a, const int tile) {
    constexpr int LW = DP + 4, DQ = DP / 4, NT = DP / 16, NJ = BK / 16, NTH = 64 * NW, CPR = DP / 4;
    float *const Ks = dq_kv_tiles<DP, BK>(), *const Vs = Ks + BK * LW;

    const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, grp = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // in a scalar register: wave-uniform branches stay scalar
    const int RB = NW / a.HW;
    const int per_tile = a.n_head_blocks * a.B;
    const int rem = (int)blockIdx.x % per_tile;
    const int hb = rem % a.n_head_blocks, b = rem / a.n_head_blocks;
    const int group = a.H / a.Hkv;
    const int h = hb * a.HW + (w % a.HW);
    const int kvh = ZT_PLANT == 12 ? 0 : h / group;
    const int wg_row0 = tile * 16 * RB;
    const int row0 = wg_row0 + 16 * (w / a.HW);
    const bool vec4 = (a.dim & 3) == 0;
    const size_t qld = (size_t)a.H * a.dim, kld = (size_t)a.Hkv * a.dim;
    const size_t qoff = (size_t)b * a.T * qld + (size_t)h * a.dim;
    const float *kb = a.k + (size_t)b * a.T * kld + (size_t)kvh * a.dim;
    const float *vb = a.v + (size_t)b * a.T * kld + (size_t)kvh * a.dim;

    const int my_row = row0 + l16;
    const bool row_ok = my_row < a.T;
    float qr[DQ], dor[DQ];
    load_row_seg<DQ>(qr, a.q + qoff + (size_t)my_row * qld, grp * DQ, a.dim, vec4, row_ok,
                     ZT_PLANT == 14 ? kLog2e : a.scale_log2e);
    load_row_seg<DQ>(dor, a.dout + qoff + (size_t)my_row * qld, grp * DQ, a.dim, vec4, row_ok, 1.f);
    float delta, lse2;
    {
        float orow[DQ];
        load_row_seg<DQ>(orow, a.o + qoff + (size_t)my_row * qld, grp * DQ, a.dim, vec4, row_ok, 1.f);
        float part = 0.f;
#pragma unroll
        for (int i = 0; i < DQ; ++i) part += orow[i] * dor[i];
        delta = sum4grp(part);
        const size_t so = ((size_t)b * a.T + my_row) * a.H + h;
        lse2 = row_ok ? a.lse[so] * kLog2e : 0.f;
        if (row_ok && grp == 0) a.row_del[so] = delta;
    }

    f4 acc[NT];
#pragma unroll
    for (int i = 0; i < NT; ++i) acc[i] = zero4();
    const int kend_wg = min(a.T, wg_row0 + 16 * RB);
    const int kend_w = row0 < a.T ? min(a.T, row0 + 16) : 0;

    constexpr int NPF = 2 * BK * CPR / NTH;
    static_assert((2 * BK * CPR) % NTH == 0, "prefetch split");
    f4 pf[NPF];
    // VEC (dim % 4 == 0, 16-byte aligned rows): every load unconditional and
    // in bounds, so the pieces go out between the score products -- keys past
    // T load key T - 1 (masked, P = 0) and columns past dim the row's last
    // chunk (met by Q's and dO's zero columns, or landing in dq columns never
    // stored).  Otherwise guarded loads, all at the top of the tile.
    // VEC: a thread's byte offsets within a tile's rows are fixed for the
    // kernel (rows tid / CPR + j RPN, its column): a piece is one load from the
    // tile's base plus the offset clamped (one min) to key T - 1, as in the
    // forward (d <= 128: C3 dq kernels 2.045 -> 2.035 ms; at d = 256 the
    // statistics-building one spills more and loses, 1.28 -> 1.32 ms).
    constexpr int RPN = NTH / CPR;
    constexpr int NOFF = DP <= 128 && (BK * CPR) % NTH == 0 && BK % RPN == 0 ? BK / RPN : 1;
    unsigned voff[NOFF];
    const unsigned coff = (unsigned)min((tid % CPR) * 4, a.dim - 4) * 4u;
#pragma unroll
    for (int j = 0; j < NOFF; ++j) voff[j] = (unsigned)((tid / CPR + j * RPN) * (int)kld) * 4u + coff;
    auto fetch_piece = [&](int n, int k0) {
        const int e = tid + n * NTH;
        const int arr = e / (BK * CPR), r = (e / CPR) % BK, c = (e % CPR) * 4;
        if constexpr (VEC && NOFF > 1) {
            // Key T - 1, counted within the tile (no 32-bit overflow however long T is).
            const unsigned last = (unsigned)(min(a.T - 1 - k0, BK - 1) * (int)kld) * 4u + coff;
            const unsigned off = min(voff[(n * RPN % BK) / RPN], last);
            pf[n] = *reinterpret_cast<const f4 *>(reinterpret_cast<const char *>((arr ? vb : kb) + (size_t)k0 * kld) + off);
        } else if constexpr (VEC) {
            pf[n] = *reinterpret_cast<const f4 *>((arr ? vb : kb) + (size_t)k0 * kld +
                                                  (min(r, a.T - 1 - k0) * (int)kld + min(c, a.dim - 4)));
        } else {
            const int key = k0 + r;
            const float *src = (arr ? vb : kb) + (size_t)key * kld + c;
            f4 x = zero4();
            if (key < a.T && c < a.dim) {
                if (vec4) {
                    x = *reinterpret_cast<const f4 *>(src);
                } else {
                    const f2 lo = *reinterpret_cast<const f2 *>(src);
                    x.x = lo.x; x.y = lo.y;
                    if (c + 2 < a.dim) {
                        const f2 hi = *reinterpret_cast<const f2 *>(src + 2);
                        x.z = hi.x; x.w = hi.y;
                    }
                }
            }
            pf[n] = x;
        }
    };
    auto fetch = [&](int k0) {
#pragma unroll
        for (int n = 0; n < NPF; ++n) fetch_piece(n, k0);
    };
    // Pieces of group i of NI between the score products (VEC, up to d = 192).
    auto fetch_group = [&](int i, int ni, int k0) {
#pragma unroll
        for (int n = i * NPF / ni; n < (i + 1) * NPF / ni; ++n) fetch_piece(n, k0);
    };
    fetch(0);

    constexpr bool ILV = VEC && DP <= 192;  // interleaved prefetch, as in bwd_dq_tile
    for (int k0 = 0; k0 < kend_wg; k0 += BK) {
        __syncthreads();
        const int kn = k0 + BK < kend_wg ? k0 + BK : k0;  // the last tile fetches itself again, unused
#pragma unroll
        for (int n = 0; n < NPF; ++n) {
            const int e = tid + n * NTH;
            const int arr = e / (BK * CPR), r = (e / CPR) % BK, c = (e % CPR) * 4;
            *reinterpret_cast<f4 *>((arr ? Vs : Ks) + r * LW + c) = pf[n];
        }
        __syncthreads();
        if constexpr (!ILV) {
            if (k0 + BK < kend_wg) fetch(k0 + BK);
        }
        if (k0 >= kend_w) {  // wave-uniform: nothing here is visible to this wave
            if constexpr (ILV) fetch(kn);
            continue;
        }

        f4 s[NJ], dp[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) { s[j] = zero4(); dp[j] = zero4(); }
        const float *krow = Ks + l16 * LW + grp * DQ;
        const float *vrow = Vs + l16 * LW + grp * DQ;
        auto score_step = [&](int j, int kk) {
            const f4 kx = *reinterpret_cast<const f4 *>(krow + 16 * j * LW + kk);
            const f4 vx = *reinterpret_cast<const f4 *>(vrow + 16 * j * LW + kk);
            s[j] = mfma16(kx.x, qr[kk + 0], s[j]);
            dp[j] = mfma16(vx.x, dor[kk + 0], dp[j]);
            s[j] = mfma16(kx.y, qr[kk + 1], s[j]);
            dp[j] = mfma16(vx.y, dor[kk + 1], dp[j]);
            s[j] = mfma16(kx.z, qr[kk + 2], s[j]);
            dp[j] = mfma16(vx.z, dor[kk + 2], dp[j]);
            s[j] = mfma16(kx.w, qr[kk + 3], s[j]);
            dp[j] = mfma16(vx.w, dor[kk + 3], dp[j]);
        };
        if constexpr (DP <= 192) {
#pragma unroll
            for (int kk = 0; kk < DQ; kk += 4) {
#pragma unroll
                for (int j = 0; j < NJ; ++j) score_step(j, kk);
                if constexpr (ILV) fetch_group(kk / 4, DQ / 4, kn);
            }
        } else {
#pragma unroll
            for (int j = 0; j < NJ; ++j)
#pragma unroll
                for (int kk = 0; kk < DQ; kk += 4) score_step(j, kk);
        }
        // dS^T[key][query] = P (dP - delta), P = exp2(S - lse2); zero where masked.
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int key = k0 + 16 * j + 4 * grp + r;
                const float e = fast_exp2(s[j][r] - lse2);
                const float p = (ZT_PLANT == 11 ? key < a.T : key <= my_row) ? e : 0.f;
                s[j][r] = ZT_PLANT == 13 ? p : p * (dp[j][r] - delta);
            }
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            if (k0 + 16 * j >= kend_w) continue;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                float kx[NT];  // K^T rows, row-owner layout
                lds_run<NT>(kx, Ks + (16 * j + 4 * grp + kk) * LW, l16);
#pragma unroll
                for (int i = 0; i < NT; ++i) acc[i] = mfma16(kx[i], s[j][kk], acc[i]);
            }
        }
    }

    if (row_ok) {
        float *dqrow = a.dq + qoff + (size_t)my_row * qld;
#pragma unroll
        for (int r = 0; r < 4; ++r) store_run<NT>(dqrow, 4 * grp + r, a.dim, vec4, acc, r, ZT_PLANT == 14 ? 1.f : a.scale);
    }
}

// DS = 2 (d-split, score-reading kernel for wide heads): a wave keeps half of
// the head's columns -- its half of V and of the dK/dV accumulators -- so two
// waves fit per SIMD; the partner wave holding the other half (w ^ KW*HS)
// shares the partial dP through LDS, both form dP = own + partner (f32
// addition commutes: the two copies are identical) and the same P and dS.
template <int DP, int HS, int KW, bool PF = false, int NU = 1, bool SIN = false, int DS = 1>
__device__ __forceinline__ void bwd_dkdv_tile(const BwdArgs &a, const int ktile, const bool up) {
    static_assert(!SIN || PF, "the scores are prefetched with the stage's rows");
    static_assert(DS == 1 || (PF && DS == 2 && (DP / 32) % 2 == 0), "d-split: prefetching, whole 32-column halves");
    constexpr int LW = DP + 4, NTH = 64 * KW * HS * DS;
    constexpr int DPW = DP / DS, DQW = DPW / 4, NTW = DPW / 16;  // a wave's columns
    constexpr int BQ = 16 * NU;  // query rows per stage: NU sub-tiles of 16
    // Per head-split part: Q rows, dO rows, and the rows' m2, -delta and 1/l
    // (BQ floats each, so that a lane reads its four rows' values as one float4).
    // With the register prefetch (PF) two such stage buffers: stage s reads one
    // while the prefetched rows of stage s + 1 are written to the other at its
    // end, one barrier per stage (C3, scores read: 1.83 -> 1.80 ms; forming S
    // again: 2.30 -> 2.23 ms).  The buffer is reused at the end for the
    // head-split sum ((HS-1) parts x KW blocks x 64 lanes x 2*NT float4).
    constexpr int STAGE_F = 2 * HS * BQ * LW + HS * BQ * 4;
    constexpr int RED_F = (HS - 1) * KW * DS * 64 * 2 * NTW * 4;
    constexpr int BUF_F = PF ? 2 * STAGE_F : STAGE_F;
    constexpr int MAIN_F = BUF_F > RED_F ? BUF_F : RED_F;
    constexpr int XCH_F = DS > 1 ? KW * HS * DS * NU * 64 * 4 * (SIN ? 1 : 2) : 0;  // partial S, dP exchange (d-split)
    __shared__ float smem[MAIN_F + XCH_F];
    float *Qs = smem, *Ds = smem + HS * BQ * LW, *St = smem + 2 * HS * BQ * LW;

    const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, grp = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // in a scalar register: wave-uniform branches stay scalar
    const int kbw = w % KW, hs = (w / KW) % HS, dh = w / (KW * HS);  // dh: the wave's column half (DS = 2)
    // Column block of the dP / S products (a lane per staged row, lane group grp
    // reading 32 of the DP columns): grp with its two bits swapped, so that
    // the lane groups a 128-bit LDS read serves together sit 64 columns (all
    // 64 banks) apart.  With grp itself the reads of rows l16 and l16 - 8 of
    // groups 0 and 1 meet in one bank: a probe of the bank-conflict counter
    // on gfx950 shows 3.8 conflict cycles per read, and none with the swap
    // (C3 dk/dv 1.776 -> 1.762 ms).  Needs DP % 128 == 0; only where the
    // scores are read (the kernel that forms S again reads Q and dO this way
    // too, and measured 2.268 -> 2.281 ms with the swap).  The dV / dK reads
    // (a lane per 16-byte chunk of rows 4 grp + kk) keep 3.8: no ownership of
    // chunks free of per-step address arithmetic removes them under every
    // lane grouping the probe admits, and an XOR-swizzled layout that does
    // cost more in registers and VALU than it saved (1.78 -> 1.81 ms).
    constexpr bool PERM = SIN && DS == 1 && DP % 128 == 0;
    const int cbk = PERM ? ((grp & 1) << 1) | (grp >> 1) : grp;
    const int per_tile = a.Hkv * a.B;
    const int rem = (int)blockIdx.x % per_tile;
    const int kvh = rem % a.Hkv, b = rem / a.Hkv;
    const int group = a.H / a.Hkv;
    const int hpp = group / HS;  // heads per part
    const int wg_s0 = ktile * 16 * KW;
    const int s0 = wg_s0 + 16 * kbw;
    const bool vec4 = (a.dim & 3) == 0;
    const size_t qld = (size_t)a.H * a.dim, kld = (size_t)a.Hkv * a.dim;
    const size_t kvoff = (size_t)b * a.T * kld + (size_t)kvh * a.dim;
    const size_t kvrd = ZT_PLANT == 12 ? (size_t)b * a.T * kld : kvoff;  // where K and V are read

    const int my_key = s0 + l16;
    const bool key_ok = my_key < a.T;
    float kr[SIN ? 1 : DQW], vr[DQW];  // with the forward's scores K is not needed
    if constexpr (!SIN)
        load_row_seg<DQW>(kr, a.k + kvrd + (size_t)my_key * kld + dh * DPW, cbk * DQW, a.dim - dh * DPW, vec4, key_ok,
                          ZT_PLANT == 14 ? kLog2e : a.scale_log2e);
    load_row_seg<DQW>(vr, a.v + kvrd + (size_t)my_key * kld + dh * DPW, cbk * DQW, a.dim - dh * DPW, vec4, key_ok,
                      1.f);

    f4 dka[NTW], dva[NTW];
#pragma unroll
    for (int i = 0; i < NTW; ++i) { dka[i] = zero4(); dva[i] = zero4(); }

    // Stages: (row tile t0 of the suffix t >= wg_s0, head of each part hi),
    // heads inner.  A workgroup's first key tile walks the rows from the last
    // one down, its partner tile (up) from the diagonal to the end: the
    // workgroups resident at one time then stand on the same row at the same
    // time in either phase and read the same Q/dO rows from L2.
    const int n_t = (a.T - wg_s0 + BQ - 1) / BQ;
    const int n_stage = hpp * n_t;
    // Tile blocks of this workgroup's (sequence, head part) in the triangular dS layout.
    const int nt16 = (a.T + 15) >> 4;
    const size_t tri_cnt = (size_t)zt_tri_count(nt16);
    const size_t hblk0 = ((size_t)b * a.H + kvh * group + hs * hpp) * tri_cnt;
    // A stage: head hi and first row t0, kept by the stage loop as it steps (no
    // division per stage), and the addresses its fetches and stores derive
    // from, formed once per stage in scalar registers.
    struct StageAt {
        int hi, t0;
        size_t roff;    // element offset of row t0, head hi of part 0 (q and dout alike)
        unsigned last;  // byte offset within the stage of its last row below T
        size_t sblk;    // first tile of head hi's dS block (this wave's part)
    };
    auto stage_at = [&](int hi, int ri) {
        const int t0 = wg_s0 + (up ? ri : n_t - 1 - ri) * BQ;
        // The offset of the last row is counted within the stage: no 32-bit overflow however long T is.
        return StageAt{hi, t0, ((size_t)b * a.T + t0) * qld + (size_t)(kvh * group + hi) * a.dim,
                       (unsigned)(min(a.T - 1 - t0, BQ - 1) * (int)qld) * 4u, hblk0 + (size_t)hi * tri_cnt};
    };
    const size_t part_off = (size_t)hpp * a.dim;  // from one part's head to the next part's

    // Register prefetch (PF): thread tid holds float4 chunks e = tid + n * NTH
    // of the stage's HS x {Q, dO} x BQ x DP block, each lane of every wave
    // one row's statistics, and each wave its score tiles (SIN); they are
    // loaded while the previous stage computes and written to LDS after the
    // next barrier.  Every load is unconditional and in bounds, so the pieces
    // can be issued between the products: rows past T load row T - 1 and
    // columns past dim the row's last four floats (the host requires dim % 4
    // == 0 and 16-byte aligned q and dout), finite values that the causal
    // mask (p = dS = 0 on rows past T) or the zero columns of K and V keep out
    // of every stored result.  The statistics stay as loaded until put():
    // arithmetic on them at the fetch would wait for the fetch's every load.
    constexpr int CPR = DP / 4;
    constexpr int NPF = PF ? HS * 2 * BQ * CPR / NTH : 1;
    static_assert(!PF || (HS * 2 * BQ * CPR) % NTH == 0, "prefetch split");
    static_assert(!PF || HS * BQ <= 64, "one wave's lanes hold a stage's row statistics");
    f4 pf[NPF];
    float pm2 = 0.f, pil = 0.f, pde = 0.f;
    bool prow = false;                      // the statistics' row is below T
    f4 sn[SIN ? NU : 1];  // the score tiles of the next stage to run (SIN)
    // A thread's byte offsets within a stage's rows, fixed for the kernel
    // (rows r = tid / CPR + j RPN of the stage, its column c): with the
    // stage's base in scalar registers a piece is one load from base + offset,
    // the offset clamped (one min) to the stage's last row below T (C3 dk/dv
    // reading scores 1.753 -> 1.729 ms, forming S again 2.271 -> 2.248 ms).
    constexpr int RPN = NTH / CPR;
    constexpr int NOFF = PF && (BQ * CPR) % NTH == 0 && BQ % RPN == 0 ? BQ / RPN : 1;
    unsigned voff[NOFF];
    const unsigned coff = (unsigned)min((tid % CPR) * 4, a.dim - 4) * 4u;
#pragma unroll
    for (int j = 0; j < NOFF; ++j) voff[j] = (unsigned)((tid / CPR + j * RPN) * (int)qld) * 4u + coff;
    auto fetch_piece = [&](int n, const StageAt x) {
        const int hi = x.hi, t0 = x.t0;
        const int e = tid + n * NTH;
        // With whole (part, array) blocks per piece, the piece's block follows
        // from n alone (tid < NTH): the base stays in scalar registers.
        const int eb = NOFF > 1 ? n * NTH : e;
        const int part = eb / (2 * BQ * CPR), arr = (eb / (BQ * CPR)) & 1;
        const float *base = (arr ? a.dout : a.q) + x.roff + part * part_off;
        (void)hi;
        if constexpr (NOFF > 1) {
            const unsigned off = min(voff[(n * RPN % BQ) / RPN], x.last + coff);  // row T - 1 at most
            pf[n] = *reinterpret_cast<const f4 *>(reinterpret_cast<const char *>(base) + off);
        } else {
            const int r = min((e / CPR) % BQ, a.T - 1 - t0), c = min((e % CPR) * 4, a.dim - 4);
            pf[n] = *reinterpret_cast<const f4 *>(base + (r * (int)qld + c));
        }
    };
    // The stage's row statistics, one row per lane of wave 0 (the wave that stores them).
    auto fetch_stats = [&](const StageAt x) {
        if (w != 0) return;  // wave-uniform
        const int hi = x.hi, t0 = x.t0;
        const int part = (lane / BQ) % HS, r = lane % BQ;
        prow = t0 + r < a.T;
        const size_t o = ((size_t)b * a.T + min(t0 + r, a.T - 1)) * a.H + kvh * group + part * hpp + hi;
        pm2 = (a.lse ? a.lse : a.row_max)[o];
        pil = (a.lse ? a.row_del : a.row_den)[o];  // unused with lse
        pde = a.row_del[o];
    };
    auto fetch_scores = [&](const StageAt x) {
        const int hi = x.hi, t0 = x.t0;
        if constexpr (SIN) {
            // This wave's score tiles of the stage (lane order, as dS is stored).
            // A tile with no visible pair (past T, above the diagonal or past
            // the last key) loads an in-bounds tile whose values the mask drops.
            const int sb = min(s0, a.T - 1) >> 4;
#pragma unroll
            for (int u = 0; u < NU; ++u) {
                const int tb = min(t0 + 16 * u, a.T - 1) >> 4;
                sn[u] = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(
                    reinterpret_cast<const char *>(a.ds_out + (x.sblk + zt_tri_index(tb, min(sb, tb))) * 256) +
                    lane * 16u));
            }
        }
        (void)hi; (void)t0;
    };
    auto fetch_aux = [&](const StageAt x) {
        fetch_stats(x);
        fetch_scores(x);
    };
    auto fetch = [&](const StageAt x) {
        fetch_aux(x);
#pragma unroll
        for (int n = 0; n < NPF; ++n) fetch_piece(n, x);
    };
    auto put = [&](int off) {
#pragma unroll
        for (int n = 0; n < NPF; ++n) {
            const int e = tid + n * NTH;
            const int part = e / (2 * BQ * CPR), arr = (e / (BQ * CPR)) & 1;
            const int r = (e / CPR) % BQ, c = (e % CPR) * 4;
            *reinterpret_cast<f4 *>((arr ? Ds : Qs) + off + (part * BQ + r) * LW + c) = pf[n];
        }
        if (tid < HS * BQ) {  // rows past T: m2 = 0, 1/l = 0, delta = 0
            float *sr = St + off + (tid / BQ) * 4 * BQ + tid % BQ;
            sr[0] = prow ? pm2 * kLog2e : 0.f;
            sr[BQ] = prow ? -pde : 0.f;
            sr[2 * BQ] = prow ? (a.lse ? 1.f : 1.f / pil) : 0.f;
        }
    };
    if constexpr (PF) fetch(stage_at(0, 0));

    // A stage's staged rows and statistics for this wave's part: with the
    // register prefetch (PF) stage stg sits in buffer stg & 1.
    auto stage_off = [&](int stg) { return PF ? (stg & 1) * STAGE_F : 0; };
    // Wave-uniform: stage stg holds a visible (query, key) pair for this wave.
    auto visible = [&](const StageAt x) { return !(x.t0 + BQ - 1 < s0 || s0 >= a.T); };

    // The first half of a visible stage's products: dP (and S again without
    // the forward's scores), then P and dS = P (dP - delta) into p and dsv,
    // and dS stored for the dq product.  The prefetch of stage nx goes out
    // between the products (PF).
    auto front = [&](int stg, const StageAt cur, const StageAt nx, f4 (&p)[NU], f4 (&dsv)[NU]) {
        const int t0 = cur.t0;
        const float *qs = Qs + stage_off(stg) + hs * BQ * LW, *ds = Ds + stage_off(stg) + hs * BQ * LW;
        const float *st = St + stage_off(stg) + hs * 4 * BQ;
        // The prefetch pieces go out between the first products' groups (the
        // next stage's scores after this stage's have been used).
        constexpr int NI = DQW / 4;
        auto fetch_after = [&](int i) {
            if constexpr (PF) {
                if (i == 0) fetch_stats(nx);
#pragma unroll
                for (int n = i * NPF / NI; n < (i + 1) * NPF / NI; ++n) fetch_piece(n, nx);
            }
        };

        // Sub-tile u holds query rows t0 + 16 u + [0, 16); this lane's four
        // rows 4 grp + r: m2 and 1/l (read ahead of the MFMAs), and -delta as
        // the dP accumulator's start, so that the products leave dP - delta
        // (d-split: in one of the two partial sums).  With the forward's scores
        // 1/l is 1 and not read.
        f4 m2v[NU], ilv[NU], s[NU], dp[NU];
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            m2v[u] = *reinterpret_cast<const f4 *>(st + 16 * u + 4 * grp);
            ilv[u] = SIN ? f4{1.f, 1.f, 1.f, 1.f} : *reinterpret_cast<const f4 *>(st + 2 * BQ + 16 * u + 4 * grp);
            dp[u] = DS == 1 || dh == 0 ? *reinterpret_cast<const f4 *>(st + BQ + 16 * u + 4 * grp) : zero4();
            s[u] = zero4();
        }
        if constexpr (SIN) {
            // Scores from the forward; dP alone, as one chain per sub-tile with
            // the sub-tiles' products interleaved (NU >= 2), else as two chains
            // summed.  (Raising the second head half's wave priority through dP,
            // so that the two waves of a SIMD leave it at different times, once
            // gained 1%; with the dP column blocks of lane groups 1 and 2 swapped
            // it costs 0.9%.)
            constexpr bool TWO = NU < 2;
            f4 dp2[NU];
#pragma unroll
            for (int u = 0; u < NU; ++u) { s[u] = sn[u]; dp2[u] = zero4(); }
            // dO operands read one group ahead of their products.
            const float *dsw = ds + dh * DPW + cbk * DQW;
            f4 dxn[NU];
#pragma unroll
            for (int u = 0; u < NU; ++u) dxn[u] = *reinterpret_cast<const f4 *>(dsw + (16 * u + l16) * LW);
#pragma unroll
            for (int kk = 0; kk < DQW; kk += 4) {
                f4 dx[NU];
#pragma unroll
                for (int u = 0; u < NU; ++u) {
                    dx[u] = dxn[u];
                    if (kk + 4 < DQW) dxn[u] = *reinterpret_cast<const f4 *>(dsw + (16 * u + l16) * LW + kk + 4);
                }
                __builtin_amdgcn_sched_barrier(0);  // keeps the reads ahead of this group's products
                if constexpr (TWO) {
#pragma unroll
                    for (int u = 0; u < NU; ++u) {
                        dp[u] = mfma16(dx[u].x, vr[kk + 0], dp[u]);
                        dp2[u] = mfma16(dx[u].y, vr[kk + 1], dp2[u]);
                        dp[u] = mfma16(dx[u].z, vr[kk + 2], dp[u]);
                        dp2[u] = mfma16(dx[u].w, vr[kk + 3], dp2[u]);
                    }
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c)
#pragma unroll
                        for (int u = 0; u < NU; ++u) dp[u] = mfma16(dx[u][c], vr[kk + c], dp[u]);
                }
                fetch_after(kk / 4);
            }
            if constexpr (TWO) {
#pragma unroll
                for (int u = 0; u < NU; ++u) dp[u] += dp2[u];
            }
            if constexpr (DS > 1) {
                float *xch = smem + MAIN_F;
#pragma unroll
                for (int u = 0; u < NU; ++u) reinterpret_cast<f4 *>(xch)[(w * NU + u) * 64 + lane] = dp[u];
                __syncthreads();
                const int pw = w ^ (KW * HS);
#pragma unroll
                for (int u = 0; u < NU; ++u) dp[u] += reinterpret_cast<const f4 *>(xch)[(pw * NU + u) * 64 + lane];
            }
        } else {
#pragma unroll
            for (int kk = 0; kk < DQW; kk += 4) {
#pragma unroll
                for (int u = 0; u < NU; ++u) {
                    const int col = dh * DPW + cbk * DQW + kk;
                    const f4 qx = *reinterpret_cast<const f4 *>(qs + (16 * u + l16) * LW + col);
                    const f4 dx = *reinterpret_cast<const f4 *>(ds + (16 * u + l16) * LW + col);
                    s[u] = mfma16(qx.x, kr[kk + 0], s[u]);
                    dp[u] = mfma16(dx.x, vr[kk + 0], dp[u]);
                    s[u] = mfma16(qx.y, kr[kk + 1], s[u]);
                    dp[u] = mfma16(dx.y, vr[kk + 1], dp[u]);
                    s[u] = mfma16(qx.z, kr[kk + 2], s[u]);
                    dp[u] = mfma16(dx.z, vr[kk + 2], dp[u]);
                    s[u] = mfma16(qx.w, kr[kk + 3], s[u]);
                    dp[u] = mfma16(dx.w, vr[kk + 3], dp[u]);
                }
                fetch_after(kk / 4);
            }
            if constexpr (DS > 1) {  // partial S and dP from the partner holding the other columns
                f4 *xch = reinterpret_cast<f4 *>(smem + MAIN_F);
#pragma unroll
                for (int u = 0; u < NU; ++u) {
                    xch[((w * NU + u) * 2 + 0) * 64 + lane] = s[u];
                    xch[((w * NU + u) * 2 + 1) * 64 + lane] = dp[u];
                }
                __syncthreads();
                const int pw = w ^ (KW * HS);
#pragma unroll
                for (int u = 0; u < NU; ++u) {
                    s[u] += xch[((pw * NU + u) * 2 + 0) * 64 + lane];
                    dp[u] += xch[((pw * NU + u) * 2 + 1) * 64 + lane];
                }
            }
        }
        // s[u][r] = S[t = t0 + 16 u + 4 grp + r][key = s0 + l16], dp[u][r] = dP - delta there.
        // With the forward's scores (log-sum-exp statistics) 1/l is 1.
        if (t0 >= s0 + 15 && t0 + BQ <= a.T) {  // wave-uniform: every pair of the stage is visible
#pragma unroll
            for (int u = 0; u < NU; ++u)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    p[u][r] = SIN ? fast_exp2(s[u][r] - m2v[u][r]) : fast_exp2(s[u][r] - m2v[u][r]) * ilv[u][r];
                    dsv[u][r] = ZT_PLANT == 13 ? p[u][r] : p[u][r] * dp[u][r];
                }
        } else {
#pragma unroll
            for (int u = 0; u < NU; ++u)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = t0 + 16 * u + 4 * grp + r;
                    const bool vis = (t < a.T) && (ZT_PLANT == 11 || t >= my_key);
                    const float e = SIN ? fast_exp2(s[u][r] - m2v[u][r]) : fast_exp2(s[u][r] - m2v[u][r]) * ilv[u][r];
                    p[u][r] = vis ? e : 0.f;
                    dsv[u][r] = ZT_PLANT == 13 ? p[u][r] : p[u][r] * dp[u][r];
                }
        }
        if constexpr (PF) fetch_scores(nx);  // this stage's scores are used: the next stage's go out
        // dS for a dq product outside this kernel, one 16 x 16 tile per (u) in lane
        // order; nontemporal, so the 1 GB stream does not evict the Q/dO rows
        // the other workgroups are about to reread.
        if (a.ds_out && dh == 0) {  // d-split: the partners hold the same dS; one stores it
#pragma unroll
            for (int u = 0; u < NU; ++u) {
                // wave-uniform: a sub-tile past the last row or above the diagonal has no slot
                if (t0 + 16 * u >= a.T || t0 + 16 * u + 15 < s0) continue;
                // (ZT_PLANT 15 swaps the two sub-tiles' slots where both exist.)
                const int us = (ZT_PLANT == 15 && NU == 2 && t0 + 16 < a.T && t0 + 15 >= s0) ? NU - 1 - u : u;
                const size_t tile = cur.sblk + zt_tri_index((t0 >> 4) + us, s0 >> 4);
                // Scalar tile base plus the lane's 32-bit byte offset.
                __builtin_nontemporal_store(
                    dsv[u], reinterpret_cast<f4 *>(reinterpret_cast<char *>(a.ds_out + tile * 256) + lane * 16u));
            }
        }
    };

    // The second half: dV^T += dO^T P and dK^T += Q^T dS from the stage's rows.
    // mid: the scalar bookkeeping of the stage after next, placed among the
    // products (at the loop's head it ran beside no MFMA).
    auto back = [&](int stg, const StageAt cur, const f4 (&p)[NU], const f4 (&dsv)[NU], auto &&mid) {
        const int t0 = cur.t0;
        const float *qs = Qs + stage_off(stg) + hs * BQ * LW, *ds = Ds + stage_off(stg) + hs * BQ * LW;
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            if (u == 1) mid();
            if (t0 + 16 * u + 15 < s0) continue;  // wave-uniform: this sub-tile is wholly masked
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                float dx[NTW], qx[NTW];  // dO^T, Q^T rows in the row-owner layout (the wave's columns)
                lds_run<NTW>(dx, ds + (16 * u + 4 * grp + kk) * LW + dh * DPW, l16);
                lds_run<NTW>(qx, qs + (16 * u + 4 * grp + kk) * LW + dh * DPW, l16);
                const float pv = p[u][kk], dv = dsv[u][kk];
#pragma unroll
                for (int i = 0; i < NTW; ++i) {
                    dva[i] = mfma16(dx[i], pv, dva[i]);
                    dka[i] = mfma16(qx[i], dv, dka[i]);
                }
            }
        }
    };

    // One whole stage: the first half, then the second.
    auto work = [&](int stg, const StageAt cur, const StageAt nx, auto &&mid) {
        if (!visible(cur)) {
            if constexpr (PF) fetch(nx);
            if constexpr (DS > 1) __syncthreads();  // the partial-dP exchange's barrier, met by every wave
            mid();
            return;
        }
        f4 p[NU], dsv[NU];
        front(stg, cur, nx, p, dsv);
        back(stg, cur, p, dsv, mid);
        if constexpr (NU < 2) mid();
    };

    if constexpr (PF) {
        put(0);
        __syncthreads();
    }
    int shi = 0, sri = 0;  // the head and row tile of the stage after the current one
    if (n_stage > 1 && ++shi == hpp) { shi = 0; ++sri; }
    StageAt cur = stage_at(0, 0), nx = n_stage > 1 ? stage_at(shi, sri) : cur;
    for (int stg = 0; stg < n_stage; ++stg) {
        // The stage after nx, formed while this stage computes (the last stages
        // fetch their own rows again, unused).
        StageAt nn = nx;
        auto mid = [&]() {
            if (stg + 2 < n_stage) {
                if (++shi == hpp) { shi = 0; ++sri; }
                nn = stage_at(shi, sri);
            }
        };
        if constexpr (!PF) {
            __syncthreads();
            const int hi = cur.hi, t0 = cur.t0;
            // Stage Q, dO rows [t0, t0+16) for every part's head.
            const int nvalid = min(BQ, a.T - t0);
            for (int part = 0; part < HS; ++part) {
                const int hh = kvh * group + part * hpp + hi;
                const size_t off = (size_t)b * a.T * qld + (size_t)t0 * qld + (size_t)hh * a.dim;
                stage_rows<DP, LW, NTH>(Qs + part * BQ * LW, a.q + off, qld, BQ, nvalid, a.dim, vec4, tid);
                stage_rows<DP, LW, NTH>(Ds + part * BQ * LW, a.dout + off, qld, BQ, nvalid, a.dim, vec4, tid);
            }
            if (tid < HS * BQ) {
                const int part = tid / BQ, r = tid % BQ, t = t0 + r;
                const int hh = kvh * group + part * hpp + hi;
                float m2 = 0.f, il = 0.f, de = 0.f;
                if (t < a.T) {
                    const size_t o = ((size_t)b * a.T + t) * a.H + hh;
                    m2 = (a.lse ? a.lse[o] : a.row_max[o]) * kLog2e;
                    il = a.lse ? 1.f : 1.f / a.row_den[o];
                    de = -a.row_del[o];
                }
                // Per part: m2, -delta and 1/l, each BQ rows long.
                St[part * 4 * BQ + r] = m2;
                St[part * 4 * BQ + BQ + r] = de;
                St[part * 4 * BQ + 2 * BQ + r] = il;
            }
            __syncthreads();
        }
        work(stg, cur, nx, mid);
        cur = nx;
        nx = nn;
        if constexpr (PF) {
            if (stg + 1 < n_stage) put(((stg + 1) & 1) * STAGE_F);
            __syncthreads();
        }
    }

    // Sum the head-split partials in a fixed order (part 0 + 1 + ...).
    if constexpr (HS > 1) {
        float *red = smem;  // (HS-1) parts x DS halves x KW blocks x 64 lanes x 2*NTW f4
        __syncthreads();
        if (hs > 0) {
            f4 *dst = reinterpret_cast<f4 *>(red) + ((((hs - 1) * DS + dh) * KW + kbw) * 64 + lane) * 2 * NTW;
#pragma unroll
            for (int i = 0; i < NTW; ++i) { dst[i] = dka[i]; dst[NTW + i] = dva[i]; }
        }
        __syncthreads();
        if (hs == 0) {
            for (int part = 1; part < HS; ++part) {
                const f4 *src =
                    reinterpret_cast<const f4 *>(red) + ((((part - 1) * DS + dh) * KW + kbw) * 64 + lane) * 2 * NTW;
#pragma unroll
                for (int i = 0; i < NTW; ++i) { dka[i] += src[i]; dva[i] += src[NTW + i]; }
            }
        }
    }
    if (hs == 0 && key_ok) {
        float *dkrow = a.dk + kvoff + (size_t)my_key * kld + dh * DPW;
        float *dvrow = a.dv + kvoff + (size_t)my_key * kld + dh * DPW;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            store_run<NTW>(dkrow, 4 * grp + r, a.dim - dh * DPW, vec4, dka, r, ZT_PLANT == 14 ? 1.f : a.scale);
            store_run<NTW>(dvrow, 4 * grp + r, a.dim - dh * DPW, vec4, dva, r, 1.f);
        }
    }
}

// dk/dv with asynchronous staging: the Q/dO rows of stage s+1 stream into the
// other half of a double-buffered LDS tile (dma16, no registers) while stage s
// computes, with one barrier per stage.  Requires dim == DP (every chunk of a
// row is inside the head) and 16-byte aligned q/dout; the host falls back to
// bwd_dkdv_body otherwise.  Same arithmetic as bwd_dkdv_body; with SIN it reads
// the forward's scores from the dS tiles as bwd_dkdv_body does.
// RS (row split, for head groups that cannot be split): the HS parts take
// alternate 16-row tiles of the same head instead of different heads, with
// four key blocks, so a workgroup runs 4 x HS waves; the parts' partial dk/dv
// are summed as the head halves' are.
template <int DP, int HS, bool SIN = false, bool RS = false>
__device__ __forceinline__ void bwd_dkdv_dma_tile(const BwdArgs &a, const int ktile) {
    static_assert(!RS || HS == 2, "row split: two parts");
    constexpr int DQ = DP / 4, NT = DP / 16, KW = RS ? 4 : 4 / HS, BQ = 16, NW = KW * HS;
    constexpr int CPR = DP / 4;          // 16-byte chunks per row
    constexpr int TILE = BQ * DP;        // floats per (part, array) tile
    constexpr int NI = BQ * CPR / 64;    // dma16 wave-instructions per tile
    constexpr int STAGE = HS * 2 * TILE; // floats per buffer
    __shared__ __attribute__((aligned(16))) float smem[2 * STAGE + 2 * HS * BQ * 4];
    float *const stats = smem + 2 * STAGE;
    static_assert((HS - 1) * KW * 64 * 2 * NT * 4 <= 2 * STAGE, "reduction buffer");

    const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, grp = lane >> 4, w = tid >> 6;
    const int kbw = w % KW, hs = w / KW;
    const int per_tile = a.Hkv * a.B;
    const int rem = (int)blockIdx.x % per_tile;
    const int kvh = rem % a.Hkv, b = rem / a.Hkv;
    const int group = a.H / a.Hkv;
    const int hpp = RS ? group : group / HS;
    const int wg_s0 = ktile * 16 * KW;
    const int s0 = wg_s0 + 16 * kbw;
    const size_t qld = (size_t)a.H * DP, kld = (size_t)a.Hkv * DP;
    const size_t kvoff = (size_t)b * a.T * kld + (size_t)kvh * DP;
    const size_t qbat = (size_t)b * a.T * qld;

    const int my_key = s0 + l16;
    const bool key_ok = my_key < a.T;
    float kr[SIN ? 1 : DQ], vr[DQ];  // with the forward's scores K is not needed
    if constexpr (!SIN)
        load_row_seg<DQ>(kr, a.k + kvoff + (size_t)my_key * kld, grp * DQ, DP, true, key_ok, a.scale_log2e);
    load_row_seg<DQ>(vr, a.v + kvoff + (size_t)my_key * kld, grp * DQ, DP, true, key_ok, 1.f);

    f4 dka[NT], dva[NT];
#pragma unroll
    for (int i = 0; i < NT; ++i) { dka[i] = zero4(); dva[i] = zero4(); }

    const int n_t = (a.T - wg_s0 + BQ - 1) / BQ;  // 16-row tiles of the suffix
    const int n_rt = RS ? (n_t + HS - 1) / HS : n_t;  // row-tile groups per head (RS: one tile per part)
    const int n_stage = hpp * n_rt;                // times the heads of a part
    // Part `part` of a stage (head hi of the part, row group rj): its head,
    // first row, and whether it has rows (RS: the last group can leave a part
    // without a tile; its copies and statistics then repeat the last tile and
    // it computes nothing).  The stage loop steps (hi, rj) along, with no
    // division per stage.
    struct PartRows { int hh, t0; bool ok; };
    struct StagePos { int hi, rj; };
    auto step = [&](StagePos x) {
        if (++x.rj == n_rt) { x.rj = 0; ++x.hi; }
        return x;
    };
    auto part_rows = [&](StagePos x, int part) {
        const int hi = x.hi, rj = x.rj;
        if constexpr (RS) {
            const int ri = rj * HS + part;
            return PartRows{kvh * group + hi, wg_s0 + min(ri, n_t - 1) * BQ, ri < n_t};
        } else {
            return PartRows{kvh * group + part * hpp + hi, wg_s0 + rj * BQ, true};
        }
    };

    // Issues the copies of stage `st` into buffer `buf`; the statistics go to
    // registers and are written to LDS by put_stats after the current compute.
    float sm2 = 0.f, sil = 0.f, sde = 0.f;
    f4 sn = zero4(), sc = zero4();  // this wave's score tile of the next / this stage (SIN)
    // A lane's byte offsets for its dma16 copies (j-th copy of this wave:
    // tile row r_j, swizzled chunk c_j), fixed for the kernel; a copy reads
    // row min(t0 + r_j, T - 1), i.e. the row offset clamped by one min.
    constexpr int NPW = HS * 2 * NI / NW;  // copies per wave per stage
    static_assert(HS * 2 * NI % NW == 0, "whole copies per wave");
    unsigned crow[NPW], ccol[NPW];
#pragma unroll
    for (int j = 0; j < NPW; ++j) {
        const int ii = (w + j * NW) % NI, e = ii * 64 + lane, r = e / CPR;
        crow[j] = (unsigned)(r * (int)qld) * 4u;
        ccol[j] = (unsigned)swz<CPR>(e % CPR, r) * 16u;
    }
    auto issue = [&](StagePos st, int buf) {
        if constexpr (SIN) {
            const PartRows pr = part_rows(st, hs);
            sn = zero4();
            if (pr.t0 + 15 >= s0 && s0 < a.T) {  // wave-uniform; t0 < T for every stage
                const int nt = (a.T + 15) >> 4;
                const size_t tile = ((size_t)b * a.H + pr.hh) * zt_tri_count(nt) + zt_tri_index(pr.t0 >> 4, s0 >> 4);
                sn = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(a.ds_out + tile * 256) + lane);
            }
        }
        if (tid < HS * BQ) {
            const PartRows pr = part_rows(st, tid / BQ);
            const int t = pr.t0 + tid % BQ;
            sm2 = 0.f; sil = 0.f; sde = 0.f;  // as loaded; put_stats finishes them
            if (t < a.T && pr.ok) {
                const size_t o = ((size_t)b * a.T + t) * a.H + pr.hh;
                sm2 = a.lse ? a.lse[o] : a.row_max[o];
                sil = a.lse ? 1.f : a.row_den[o];
                sde = a.row_del[o];
            }
        }
#pragma unroll
        for (int j = 0; j < NPW; ++j) {
            const int i = w + j * NW;  // wave-uniform
            const int part = i / (2 * NI), arr = (i / NI) & 1, ii = i % NI;
            const PartRows pr = part_rows(st, part);
            // Rows past T: a real row (T - 1), masked below.
            const char *src = reinterpret_cast<const char *>((arr ? a.dout : a.q) + qbat + (size_t)pr.hh * DP +
                                                             (size_t)pr.t0 * qld);
            const unsigned last = (unsigned)(min(a.T - 1 - pr.t0, BQ - 1) * (int)qld) * 4u;
            dma16(reinterpret_cast<const float *>(src + (min(crow[j], last) + ccol[j])),
                  smem + buf * STAGE + (part * 2 + arr) * TILE + ii * 256);
        }
    };
    auto put_stats = [&](int buf) {
        if (tid < HS * BQ) {
            float *sp = stats + (buf * HS * BQ + tid) * 4;
            sp[0] = sm2 * kLog2e;
            sp[1] = a.lse || sil == 0.f ? sil : 1.f / sil;  // l >= 1 on every row below T
            sp[2] = sde;
        }
    };

    StagePos pos{0, 0};
    issue(pos, 0);
    put_stats(0);
    wait_dma();
    __syncthreads();
    for (int st = 0; st < n_stage; ++st) {
        const int buf = st & 1;
        const StagePos nxt = step(pos);
        if constexpr (SIN) sc = sn;
        if (st + 1 < n_stage) issue(nxt, buf ^ 1);
        const PartRows mine = part_rows(pos, hs);
        const int t0 = mine.t0;
        if (mine.ok && !(t0 + 15 < s0 || s0 >= a.T)) {
            const float *qs = smem + buf * STAGE + (hs * 2 + 0) * TILE;
            const float *ds = smem + buf * STAGE + (hs * 2 + 1) * TILE;
            const float *sp = stats + buf * HS * BQ * 4 + hs * BQ * 4;
            f4 stv[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) stv[r] = *reinterpret_cast<const f4 *>(sp + (4 * grp + r) * 4);
            f4 s = zero4(), dp = zero4();
            if constexpr (SIN) {
                // Scores from the forward; dP alone as two interleaved chains.
                f4 dp2 = zero4();
                s = sc;
                // One wave per SIMD here: each group's dO operand is read one
                // group ahead, so no product waits for its LDS read.
                f4 dxn = *reinterpret_cast<const f4 *>(ds + l16 * DP + 4 * swz<CPR>((grp * DQ) >> 2, l16));
#pragma unroll
                for (int kk = 0; kk < DQ; kk += 4) {
                    const f4 dx = dxn;
                    if (kk + 4 < DQ)
                        dxn = *reinterpret_cast<const f4 *>(ds + l16 * DP + 4 * swz<CPR>((grp * DQ + kk + 4) >> 2, l16));
                    __builtin_amdgcn_sched_barrier(0);
                    dp = mfma16(dx.x, vr[kk + 0], dp);
                    dp2 = mfma16(dx.y, vr[kk + 1], dp2);
                    dp = mfma16(dx.z, vr[kk + 2], dp);
                    dp2 = mfma16(dx.w, vr[kk + 3], dp2);
                }
                dp += dp2;
            } else {
                f4 qxn = *reinterpret_cast<const f4 *>(qs + l16 * DP + 4 * swz<CPR>((grp * DQ) >> 2, l16));
                f4 dxn = *reinterpret_cast<const f4 *>(ds + l16 * DP + 4 * swz<CPR>((grp * DQ) >> 2, l16));
#pragma unroll
                for (int kk = 0; kk < DQ; kk += 4) {
                    const f4 qx = qxn, dx = dxn;
                    if (kk + 4 < DQ) {
                        const int off = l16 * DP + 4 * swz<CPR>((grp * DQ + kk + 4) >> 2, l16);
                        qxn = *reinterpret_cast<const f4 *>(qs + off);
                        dxn = *reinterpret_cast<const f4 *>(ds + off);
                    }
                    __builtin_amdgcn_sched_barrier(0);
                    s = mfma16(qx.x, kr[kk + 0], s);
                    dp = mfma16(dx.x, vr[kk + 0], dp);
                    s = mfma16(qx.y, kr[kk + 1], s);
                    dp = mfma16(dx.y, vr[kk + 1], dp);
                    s = mfma16(qx.z, kr[kk + 2], s);
                    dp = mfma16(dx.z, vr[kk + 2], dp);
                    s = mfma16(qx.w, kr[kk + 3], s);
                    dp = mfma16(dx.w, vr[kk + 3], dp);
                }
            }
            f4 p, dsv;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = t0 + 4 * grp + r;
                const bool vis = (t < a.T) && (t >= my_key);
                const float e = fast_exp2(s[r] - stv[r].x) * stv[r].y;
                p[r] = vis ? e : 0.f;
                dsv[r] = p[r] * (dp[r] - stv[r].z);
            }
            if (a.ds_out) {  // dS for a dq product outside this kernel: the 16 x 16 tile in lane order
                const int nt = (a.T + 15) >> 4;
                const size_t tile = ((size_t)b * a.H + mine.hh) * zt_tri_count(nt) + zt_tri_index(t0 >> 4, s0 >> 4);
                __builtin_nontemporal_store(dsv, reinterpret_cast<f4 *>(a.ds_out + tile * 256) + lane);
            }
            // dO^T, Q^T rows in the row-owner layout, read one row ahead.
            float dxn[NT], qxn[NT];
            lds_run_swz<NT, CPR>(dxn, ds, 4 * grp, l16);
            lds_run_swz<NT, CPR>(qxn, qs, 4 * grp, l16);
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const float pv = p[kk], dv = dsv[kk];
                float dx[NT], qx[NT];
#pragma unroll
                for (int i = 0; i < NT; ++i) { dx[i] = dxn[i]; qx[i] = qxn[i]; }
                if (kk + 1 < 4) {
                    lds_run_swz<NT, CPR>(dxn, ds, 4 * grp + kk + 1, l16);
                    lds_run_swz<NT, CPR>(qxn, qs, 4 * grp + kk + 1, l16);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int i = 0; i < NT; ++i) {
                    dva[i] = mfma16(dx[i], pv, dva[i]);
                    dka[i] = mfma16(qx[i], dv, dka[i]);
                }
            }
        }
        if (st + 1 < n_stage) put_stats(buf ^ 1);
        wait_dma();
        __syncthreads();
        pos = nxt;
    }

    if constexpr (HS > 1) {
        float *red = smem;
        if (hs > 0) {
            f4 *dst = reinterpret_cast<f4 *>(red) + (((hs - 1) * KW + kbw) * 64 + lane) * 2 * NT;
#pragma unroll
            for (int i = 0; i < NT; ++i) { dst[i] = dka[i]; dst[NT + i] = dva[i]; }
        }
        __syncthreads();
        if (hs == 0) {
            for (int part = 1; part < HS; ++part) {
                const f4 *src = reinterpret_cast<const f4 *>(red) + (((part - 1) * KW + kbw) * 64 + lane) * 2 * NT;
#pragma unroll
                for (int i = 0; i < NT; ++i) { dka[i] += src[i]; dva[i] += src[NT + i]; }
            }
        }
    }
    if (hs == 0 && key_ok) {
        float *dkrow = a.dk + kvoff + (size_t)my_key * kld;
        float *dvrow = a.dv + kvoff + (size_t)my_key * kld;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            store_run<NT>(dkrow, 4 * grp + r, DP, true, dka, r, a.scale);
            store_run<NT>(dvrow, 4 * grp + r, DP, true, dva, r, 1.f);
        }
    }
}

// Up to d = 192 (d = 128 with 64-key tiles, whose LDS holds one workgroup per
// CU above it) the dq kernel fits two waves per SIMD without spilling when
// asked to (four accumulator/operand sets of DP/4 registers each); above that
// it keeps one.
// Grid order and pairing.  Row tiles (dq kernels) run latest first and key
// tiles (dk/dv kernels) earliest first, heaviest first either way; with
// a.pair a workgroup also takes the partner tile at the other end (p with
// n - 1 - p), so every workgroup has the same causal work and those resident
// together end together.
template <int DP, int BK, int NW, bool PF = false, bool VEC = false>
__device__ __forceinline__ void bwd_dq_pair(const BwdArgs &a) {
    const int p = (int)blockIdx.x / (a.n_head_blocks * a.B), n = a.n_row_tiles;
    bwd_dq_tile<DP, BK, NW, PF, VEC>(a, n - 1 - p);
    if (a.pair && p < n - 1 - p) {  // workgroup-uniform
        __syncthreads();  // the first tile's last LDS reads before the second's writes
        bwd_dq_tile<DP, BK, NW, PF, VEC>(a, p);
    }
}
// The prefetching kernels take 16-byte row chunks unconditionally when dim %
// 4 == 0 (rows the library requires 16-byte aligned), guarded loads otherwise.
template <int DP, int BK, int NW, bool PF = false>
__device__ __forceinline__ void bwd_dq_body(const BwdArgs &a) {
    if constexpr (PF) {
        if ((a.dim & 3) == 0) bwd_dq_pair<DP, BK, NW, true, true>(a);
        else bwd_dq_pair<DP, BK, NW, true, false>(a);
    } else {
        bwd_dq_pair<DP, BK, NW, false, false>(a);
    }
}
template <int DP, int BK, int NW, bool VEC>
__device__ __forceinline__ void bwd_dq_lse_pair(const BwdArgs &a) {
    const int p = (int)blockIdx.x / (a.n_head_blocks * a.B), n = a.n_row_tiles;
    bwd_dq_lse_tile<DP, BK, NW, VEC>(a, n - 1 - p);
    if (a.pair && p < n - 1 - p) {
        __syncthreads();
        bwd_dq_lse_tile<DP, BK, NW, VEC>(a, p);
    }
}
template <int DP, int BK, int NW>
__device__ __forceinline__ void bwd_dq_lse_body(const BwdArgs &a) {
    if ((a.dim & 3) == 0) bwd_dq_lse_pair<DP, BK, NW, true>(a);
    else bwd_dq_lse_pair<DP, BK, NW, false>(a);
}
template <int DP, int HS, int KW, bool PF = false, int NU = 1, bool SIN = false, int DS = 1>
__device__ __forceinline__ void bwd_dkdv_body(const BwdArgs &a) {
    const int p = (int)blockIdx.x / (a.Hkv * a.B), n = a.n_key_tiles;
    bwd_dkdv_tile<DP, HS, KW, PF, NU, SIN, DS>(a, p, false);
    if (a.pair && n - 1 - p > p) {
        __syncthreads();  // the head-split sum reads LDS; the next tile's staging writes it
        bwd_dkdv_tile<DP, HS, KW, PF, NU, SIN, DS>(a, n - 1 - p, true);
    }
}
template <int DP, int HS, bool SIN = false, bool RS = false>
__device__ __forceinline__ void bwd_dkdv_dma_body(const BwdArgs &a) {
    const int p = (int)blockIdx.x / (a.Hkv * a.B), n = a.n_key_tiles;
    bwd_dkdv_dma_tile<DP, HS, SIN, RS>(a, p);
    if (a.pair && n - 1 - p > p) {
        __syncthreads();  // the head-split sum reads LDS; the next tile's copies start at once
        bwd_dkdv_dma_tile<DP, HS, SIN, RS>(a, n - 1 - p);
    }
}

#define ZT_BWD_DQ(DP, BK)                                                                          \
    extern "C" __global__ void __launch_bounds__(256, (DP) <= ((BK) == 32 ? 192 : 128) ? 2 : 1)  \
        zt_bwd_dq_d##DP##_k##BK(BwdArgs a) {                                                       \
        bwd_dq_body<DP, BK, 4>(a);                                                                 \
    }                                                                                              \
    extern "C" __global__ void __launch_bounds__(512) zt_bwd_dq8_d##DP##_k##BK(BwdArgs a) {      \
        bwd_dq_body<DP, BK, 8>(a);                                                                 \
    }
// dq from saved statistics (32-key tiles, register prefetch), four waves.
#define ZT_BWD_DQ_LSE(DP)                                                                          \
    extern "C" __global__ void __launch_bounds__(256, (DP) <= 192 ? 2 : 1)                        \
        zt_bwd_dql_d##DP##_k32(BwdArgs a) {                                                        \
        bwd_dq_lse_body<DP, 32, 4>(a);                                                             \
    }
// Register-prefetched dq (32-key tiles), four and eight waves.
#define ZT_BWD_DQ_PF(DP)                                                                           \
    extern "C" __global__ void __launch_bounds__(256, (DP) <= 192 ? 2 : 1)                        \
        zt_bwd_dqp_d##DP##_k32(BwdArgs a) {                                                        \
        bwd_dq_body<DP, 32, 4, true>(a);                                                           \
    }                                                                                              \
    extern "C" __global__ void __launch_bounds__(512) zt_bwd_dq8p_d##DP##_k32(BwdArgs a) {       \
        bwd_dq_body<DP, 32, 8, true>(a);                                                           \
    }
#define ZT_BWD_DKDV(DP, HS)                                                                        \
    extern "C" __global__ void __launch_bounds__(256) zt_bwd_dkdv_d##DP##_hs##HS(BwdArgs a) {   \
        bwd_dkdv_body<DP, HS, 4 / HS>(a);                                                          \
    }
// Eight waves: 4 key blocks x 2 head halves share each staged Q/dO tile.
#define ZT_BWD_DKDV8(DP)                                                                           \
    extern "C" __global__ void __launch_bounds__(512) zt_bwd_dkdv8_d##DP##_hs2(BwdArgs a) {     \
        bwd_dkdv_body<DP, 2, 4>(a);                                                                \
    }                                                                                              \
    extern "C" __global__ void __launch_bounds__(512) zt_bwd_dkdv8p_d##DP##_hs2(BwdArgs a) {    \
        bwd_dkdv_body<DP, 2, 4, true>(a);                                                          \
    }
// Eight-wave dk/dv that reads the forward's scores instead of recomputing Q K^T,
// 32 query rows per stage (without K in registers two 16-row sub-tiles fit:
// C3 2.09 -> 2.02 ms against one).
#define ZT_BWD_DKDV8S(DP)                                                                          \
    extern "C" __global__ void __launch_bounds__(512) zt_bwd_dkdv8s_d##DP##_hs2(BwdArgs a) {    \
        bwd_dkdv_body<DP, 2, 4, true, 2, true>(a);                                                 \
    }
#define ZT_BWD_DKDV_DMA(DP, HS)                                                                    \
    extern "C" __global__ void __launch_bounds__(256) zt_bwd_dkdv_dma_d##DP##_hs##HS(BwdArgs a) { \
        bwd_dkdv_dma_body<DP, HS>(a);                                                              \
    }
// The asynchronously staged kernel reading the forward's scores (wide heads).
#define ZT_BWD_DKDV_DMAS(DP)                                                                       \
    extern "C" __global__ void __launch_bounds__(256) zt_bwd_dkdv_dmas_d##DP##_hs2(BwdArgs a) {  \
        bwd_dkdv_dma_body<DP, 2, true>(a);                                                         \
    }
#define ZT_BWD_ALL(DP)                                                                             \
    ZT_BWD_DQ(DP, 32) ZT_BWD_DQ(DP, 64) ZT_BWD_DQ_PF(DP) ZT_BWD_DQ_LSE(DP) ZT_BWD_DKDV(DP, 1) ZT_BWD_DKDV(DP, 2) ZT_BWD_DKDV8(DP)    \
    ZT_BWD_DKDV_DMA(DP, 1) ZT_BWD_DKDV_DMA(DP, 2)

#if ZT_PLANT == 0
ZT_BWD_ALL(32)
ZT_BWD_ALL(64)
ZT_BWD_ALL(96)
ZT_BWD_ALL(128)
ZT_BWD_DKDV8S(32) ZT_BWD_DKDV8S(64) ZT_BWD_DKDV8S(96) ZT_BWD_DKDV8S(128)
// The 4-way splits: the 160 KB LDS holds 4 parts' tiles (double-buffered for
// the asynchronous variant) up to d = 128.
ZT_BWD_DKDV(32, 4)
ZT_BWD_DKDV(64, 4)
ZT_BWD_DKDV(96, 4)
ZT_BWD_DKDV(128, 4)
// Row-split asynchronously staged dk/dv (head groups that cannot be split,
// such as MHA): eight waves, 4 key blocks x 2 row parts.
#define ZT_BWD_DKDV_DMAR(DP)                                                                       \
    extern "C" __global__ void __launch_bounds__(512) zt_bwd_dkdv_dmar_d##DP(BwdArgs a) {        \
        bwd_dkdv_dma_body<DP, 2, false, true>(a);                                                  \
    }
ZT_BWD_DKDV_DMAR(32) ZT_BWD_DKDV_DMAR(64) ZT_BWD_DKDV_DMAR(96) ZT_BWD_DKDV_DMAR(128)
// The same reading the forward's scores: each part's wave loads its own
// row tile's score tile and writes dS over it.
#define ZT_BWD_DKDV_DMARS(DP)                                                                      \
    extern "C" __global__ void __launch_bounds__(512) zt_bwd_dkdv_dmars_d##DP(BwdArgs a) {       \
        bwd_dkdv_dma_body<DP, 2, true, true>(a);                                                   \
    }
ZT_BWD_DKDV_DMARS(32) ZT_BWD_DKDV_DMARS(64) ZT_BWD_DKDV_DMARS(96) ZT_BWD_DKDV_DMARS(128)
ZT_BWD_DKDV_DMA(32, 4)
ZT_BWD_DKDV_DMA(64, 4)
ZT_BWD_DKDV_DMA(96, 4)
ZT_BWD_DKDV_DMA(128, 4)
ZT_BWD_ALL(160)
ZT_BWD_ALL(192)
ZT_BWD_ALL(224)
ZT_BWD_ALL(256)
ZT_BWD_DKDV_DMAS(160) ZT_BWD_DKDV_DMAS(192) ZT_BWD_DKDV_DMAS(224) ZT_BWD_DKDV_DMAS(256)
// Score-reading dk/dv for wide heads with the head's columns split over two
// waves (DS = 2): eight waves (2 key blocks x 2 head halves x 2 column halves),
// two per SIMD, 16 query rows per stage in two buffers.  Heads whose halves
// are whole 32-column groups (d = 192, 256).
#define ZT_BWD_DKDV8SD(DP)                                                                         \
    extern "C" __global__ void __launch_bounds__(512) zt_bwd_dkdv8sd_d##DP##_hs2(BwdArgs a) {   \
        bwd_dkdv_body<DP, 2, 2, true, 1, true, 2>(a);                                              \
    }
ZT_BWD_DKDV8SD(192) ZT_BWD_DKDV8SD(256)
// The same column split for the kernel that forms S again (reference entry
// point and the training path without scores), partial S and dP exchanged;
// for groups that cannot be halved (MHA, odd groups) four key blocks x two
// column halves of one part, also at d = 64 and 128.
#define ZT_BWD_DKDV8PD(DP)                                                                         \
    extern "C" __global__ void __launch_bounds__(512) zt_bwd_dkdv8pd_d##DP##_hs2(BwdArgs a) {   \
        bwd_dkdv_body<DP, 2, 2, true, 1, false, 2>(a);                                             \
    }                                                                                              \
    extern "C" __global__ void __launch_bounds__(512) zt_bwd_dkdv8pd_d##DP##_hs1(BwdArgs a) {   \
        bwd_dkdv_body<DP, 1, 4, true, 1, false, 2>(a);                                             \
    }
ZT_BWD_DKDV8PD(192) ZT_BWD_DKDV8PD(256)
#define ZT_BWD_DKDV8PD1(DP)                                                                        \
    extern "C" __global__ void __launch_bounds__(512) zt_bwd_dkdv8pd_d##DP##_hs1(BwdArgs a) {   \
        bwd_dkdv_body<DP, 1, 4, true, 1, false, 2>(a);                                             \
    }
ZT_BWD_DKDV8PD1(64) ZT_BWD_DKDV8PD1(128)
#else
// A planted-defect build (test-only): the kernels of the negative-control
// shapes, d = 32 (the reference entry points) and d = 128 (the training path).
ZT_BWD_DQ_PF(32) ZT_BWD_DQ_LSE(32) ZT_BWD_DKDV8(32) ZT_BWD_DKDV8S(128)
#endif

// delta[row] = sum_d o[row, d] * dout[row, d] over the B*T*H rows of dim
// floats (the row statistic the dk/dv kernel needs, autograd.zig:774-797 as
// dO . O).  16 lanes per row, 4 rows per wave, 16 rows per workgroup.
extern "C" __global__ void __launch_bounds__(256) zt_bwd_delta(BwdArgs a) {
    const int lane = threadIdx.x & 63, l16 = lane & 15;
    const long long rows = (long long)a.B * a.T * a.H;
    const long long row = (long long)blockIdx.x * 16 + (threadIdx.x >> 4);
    const bool vec4 = (a.dim & 3) == 0;
    float part = 0.f;
    if (row < rows) {
        const float *o = a.o + (size_t)row * a.dim, *d = a.dout + (size_t)row * a.dim;
        for (int c = 4 * l16; c < a.dim; c += 64) {
            float x[4], y[4];
            load_row_seg<4>(x, o, c, a.dim, vec4, true, 1.f);
            load_row_seg<4>(y, d, c, a.dim, vec4, true, 1.f);
            part += (x[0] * y[0] + x[1] * y[1]) + (x[2] * y[2] + x[3] * y[3]);
        }
    }
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) part += wave_xor(part, m);
    if (row < rows && l16 == 0) a.row_del[row] = part;
}

