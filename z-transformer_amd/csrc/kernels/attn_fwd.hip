// Fused causal grouped-query attention, forward, f32 on FP32 MFMA (gfx950).
//
// Computes what src/cuda/attn_kernels.cu:197-369 (fusedAttnForward) computes
// -- O = softmax(Q K^T / sqrt(d), causal) V with query row t at absolute
// position q_offset + t seeing keys s <= q_offset + t, s < n_keys -- but with
// a different schedule:
//   * a workgroup is NW = 4 or 8 waves; each wave owns 16 query rows of one
//     query head.  The waves are HW query heads of ONE kv group x (NW / HW) row blocks,
//     so each K/V tile staged in LDS is read from HBM/L2 once per kv group
//     instead of once per query (the reference re-reads the prefix per query);
//   * Q stays in registers for the whole key loop, pre-scaled by
//     log2(e)/sqrt(d) so the softmax runs on exp2;
//   * S^T = K Q^T and O^T += V^T P^T on v_mfma_f32_16x16x4_f32, with P passed
//     register to register (layout notes in common.h);
//   * online softmax with a per-lane partial denominator that is reduced once
//     at the end; only the running max is exchanged across lanes per tile.
// The grid is 1-D, heaviest (latest) row tiles first, with the kv group as the
// fastest-varying index so that consecutive workgroups -- which the dispatcher
// spreads across the XCDs -- keep one kv group's K/V per XCD L2.
#include "common.h"
#include "args.h"


// KS > 1 (key split): the workgroup's waves are KS key parts x (NW / KS) row
// blocks; a step stages KS consecutive BK-key tiles, part kh computes with
// tile kh, each keeps its own running max, sum and output, and the parts are
// merged through LDS at the end.  KS times the waves for the same rows: on
// grids that give a four-wave workgroup per CU (one wave per SIMD, MHA at
// small batch) the other waves of a SIMD cover each one's latencies.
template <int DP, int BK, int NW, bool PF, int KS = 1>
__device__ __forceinline__ void attn_fwd_tile(const FwdArgs &a, const int tile) {
    static_assert(KS == 1 || PF, "the key split stages with the register prefetch");
    constexpr int LW = DP + 4;  // LDS row stride: +16 B spreads row starts over banks
    constexpr int DQ = DP / 4;  // d values per lane group
    constexpr int NT = DP / 16; // 16-wide column tiles of the output
    constexpr int NJ = BK / 16; // 16-key sub-blocks per LDS tile
    constexpr int NTH = 64 * NW;
    constexpr int KBK = KS * BK;  // keys staged per step
    constexpr int MRG_F = (KS - 1) * (NW / KS) * 64 * (4 * NT + 2);  // the key parts' merge
    constexpr int SM_F = 2 * KBK * LW > MRG_F ? 2 * KBK * LW : MRG_F;
    __shared__ float smem[SM_F];
    float *const Ks = smem, *const Vs = smem + KBK * LW;

    const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, grp = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // in a scalar register: wave-uniform branches stay scalar
    const int kh = w / (NW / KS);  // key part (KS > 1)
    const int wr = w % (NW / KS);  // the wave's (head, row block) slot
    const int RB = NW / KS / a.HW;  // 16-row blocks per head in this workgroup
    const int per_tile = a.n_head_blocks * a.B;
    const int rem = (int)blockIdx.x % per_tile;
    const int hb = rem % a.n_head_blocks, b = rem / a.n_head_blocks;
    const int group = a.H / a.Hkv;
    const int h = hb * a.HW + (wr % a.HW);
    const int kvh = ZT_PLANT == 2 ? 0 : h / group;
    const int wg_row0 = tile * 16 * RB;
    const int row0 = wg_row0 + 16 * (wr / a.HW);
    const bool vec4 = (a.dim & 3) == 0;
    const size_t qld = (size_t)a.H * a.dim, kld = (size_t)a.Hkv * a.dim;
    const float *qb = a.q + (size_t)b * a.T * qld + (size_t)h * a.dim;
    const float *kb = a.k + (size_t)b * a.kv_rows * kld + (size_t)kvh * a.dim;
    const float *vb = a.v + (size_t)b * a.kv_rows * kld + (size_t)kvh * a.dim;

    const int my_row = row0 + l16;
    float qr[DQ];
    load_row_seg<DQ>(qr, qb + (size_t)my_row * qld, grp * DQ, a.dim, vec4, my_row < a.T,
                     ZT_PLANT == 4 ? kLog2e : a.scale_log2e);

    f4 o[NT];
#pragma unroll
    for (int i = 0; i < NT; ++i) o[i] = zero4();
    float m = -INFINITY, lsum = 0.f;
    const int qpos = a.q_offset + my_row;
    const int kend_wg = min(a.n_keys, a.q_offset + min(a.T, wg_row0 + 16 * RB));
    const int kend_w = row0 < a.T ? min(a.n_keys, a.q_offset + min(a.T, row0 + 16)) : 0;

    // Register prefetch (PF): thread tid holds float4 chunks e = tid + n * NTH
    // of the next K/V tile (2 x BK x DP floats), loaded while the current tile
    // computes and written to LDS after the next barrier.  Every load is
    // unconditional and in bounds, so the pieces can be issued between the
    // score products: keys past n_keys load key n_keys - 1 (their scores are
    // masked, so P is 0 there) and columns past dim the row's last four floats
    // (met by Q's zero columns, or landing in output columns never stored); the
    // host picks this kernel only for dim % 4 == 0, whose rows are 16-byte aligned.
    constexpr int CPR = DP / 4;
    constexpr int NPF = PF ? 2 * KBK * CPR / NTH : 1;
    static_assert(!PF || (2 * KBK * CPR) % NTH == 0, "prefetch split");
    f4 pf[NPF];
    // A thread's byte offsets within a tile's rows (rows tid / CPR + j RPN,
    // its column), fixed for the kernel: a piece is one load from the tile's
    // base in scalar registers plus the offset clamped (one min) to key
    // n_keys - 1, with no per-piece address arithmetic (C3 training forward
    // 1.092 -> 1.066 ms, C5 0.563 -> 0.551 ms).
    constexpr int RPN = NTH / CPR;
    constexpr int NOFF = PF && (KBK * CPR) % NTH == 0 && KBK % RPN == 0 ? KBK / RPN : 1;
    unsigned voff[NOFF];
    const unsigned coff = (unsigned)min((tid % CPR) * 4, a.dim - 4) * 4u;
#pragma unroll
    for (int j = 0; j < NOFF; ++j) voff[j] = (unsigned)((tid / CPR + j * RPN) * (int)kld) * 4u + coff;
    auto fetch_piece = [&](int n, int k0) {
        const int e = tid + n * NTH;
        // With whole arrays per piece, the piece's array follows from n alone
        // (tid < NTH): the base stays in scalar registers.
        const int arr = (NOFF > 1 ? n * NTH : e) / (KBK * CPR);
        if constexpr (NOFF > 1) {
            // Key n_keys - 1, counted within the tile (no 32-bit overflow however many keys).
            const unsigned last = (unsigned)(min(a.n_keys - 1 - k0, KBK - 1) * (int)kld) * 4u + coff;
            const unsigned off = min(voff[(n * RPN % KBK) / RPN], last);
            pf[n] = *reinterpret_cast<const f4 *>(reinterpret_cast<const char *>((arr ? vb : kb) + (size_t)k0 * kld) + off);
        } else {
            const int r = min((e / CPR) % KBK, a.n_keys - 1 - k0), c = min((e % CPR) * 4, a.dim - 4);
            pf[n] = *reinterpret_cast<const f4 *>((arr ? vb : kb) + (size_t)k0 * kld + (r * (int)kld + c));
        }
    };
    auto fetch = [&](int k0) {
#pragma unroll
        for (int n = 0; n < NPF; ++n) fetch_piece(n, k0);
    };
    if constexpr (PF) fetch(0);

    for (int ks0 = 0; ks0 < kend_wg; ks0 += KBK) {
        __syncthreads();
        // The tile the prefetch loads meanwhile (the last one loads itself again, unused).
        const int kn = ks0 + KBK < kend_wg ? ks0 + KBK : ks0;
        // This wave's tile of the step: keys k0 .. k0 + BK - 1, its rows in LDS from kt.
        const int k0 = ks0 + kh * BK, kt = kh * BK * LW;
        if constexpr (PF) {
#pragma unroll
            for (int n = 0; n < NPF; ++n) {
                const int e = tid + n * NTH;
                const int arr = e / (KBK * CPR), r = (e / CPR) % KBK, c = (e % CPR) * 4;
                *reinterpret_cast<f4 *>((arr ? Vs : Ks) + r * LW + c) = pf[n];
            }
            __syncthreads();
        } else {
            const int nvalid = min(BK, a.n_keys - k0);
            stage_rows<DP, LW, NTH>(Ks, kb + (size_t)k0 * kld, kld, BK, nvalid, a.dim, vec4, tid);
            stage_rows<DP, LW, NTH>(Vs, vb + (size_t)k0 * kld, kld, BK, nvalid, a.dim, vec4, tid);
            __syncthreads();
        }
        if (k0 >= kend_w) {  // wave-uniform: nothing here is visible to this wave
            if constexpr (PF) fetch(kn);
            continue;
        }

        // Scores for every 16-key sub-block, the NJ accumulation chains
        // interleaved so consecutive MFMAs are independent.  A sub-block that is
        // wholly invisible to this wave is computed and then masked.
        f4 s[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) s[j] = zero4();
        const float *krow = Ks + kt + l16 * LW + grp * DQ;
#pragma unroll
        for (int kk = 0; kk < DQ; kk += 4) {
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const f4 kx = *reinterpret_cast<const f4 *>(krow + 16 * j * LW + kk);
                s[j] = mfma16(kx.x, qr[kk + 0], s[j]);
                s[j] = mfma16(kx.y, qr[kk + 1], s[j]);
                s[j] = mfma16(kx.z, qr[kk + 2], s[j]);
                s[j] = mfma16(kx.w, qr[kk + 3], s[j]);
            }
            if constexpr (PF) {  // the prefetch pieces go out between the score products
                constexpr int NI = DQ / 4;
#pragma unroll
                for (int n = (kk / 4) * NPF / NI; n < (kk / 4 + 1) * NPF / NI; ++n) fetch_piece(n, kn);
            }
        }
        if (a.s_out) {
            // Element (t = row0 + l16, s = k0 + 16 j + 4 grp + r) goes to lane
            // (s & 15) + 16 ((t & 15) >> 2), element t & 3 of its tile: four
            // lanes write each 16-byte run.  (A quad transpose to one 16-byte
            // store per lane measured no faster.)  Nontemporal: the 1 GB of
            // tiles would otherwise displace the K/V rows the workgroups share
            // in L2 (C3 1.100 -> 1.092 ms, C5 0.576 -> 0.563 ms).
            // Row tile row0 / 16 keeps its tiles 0..row0 / 16 contiguous, so
            // sub-block j of this key tile is j tiles after its first.
            const int nt = (a.T + 15) >> 4;
            float *srow = a.s_out + (((size_t)b * a.H + h) * zt_tri_count(nt) + zt_tri_index(row0 >> 4, k0 >> 4)) * 256 +
                          (16 * (l16 >> 2)) * 4 + (l16 & 3);
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                if (k0 + 16 * j >= kend_w) continue;  // wave-uniform: above the diagonal
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    __builtin_nontemporal_store(ZT_PLANT == 5 ? s[j][r] / a.scale_log2e : s[j][r],
                                                srow + j * 256 + (4 * grp + r) * 4);
            }
        }
        if (k0 + BK - 1 > a.q_offset + row0 || k0 + BK > a.n_keys) {  // wave-uniform: a key past a row or past n_keys
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int key = k0 + 16 * j + 4 * grp + r;
                    if ((ZT_PLANT != 1 && key > qpos) || key >= a.n_keys) s[j][r] = -INFINITY;
                }
            }
        }
        float sv[4 * NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) sv[4 * j + r] = s[j][r];
        const float mt = max4grp(vmax_n(sv));
        // Lazy rescaling: a row's exponent base m moves only when the row meets
        // a tile maximum more than 8 (log2 units) above it, so between moves
        // every exp2 stays at most 2^8 and the running sum and O need no
        // rescaling (C3 training forward 1.114 -> 1.099 ms, C5 0.587 -> 0.577 ms;
        // the rescale's 32 multiplies per tile ran beside no MFMA).  The first tile always moves it (m
        // starts at -inf; key 0 is visible to every row, so mt is finite
        // there); the result is the eager rescaling's up to rounding.  Decided
        // per row (the four lanes of a row agree), not per wave: a row's
        // arithmetic then depends on no other row, and the branch is skipped
        // when no row of the wave moves.
        if (ZT_PLANT == 3 || mt > m + 8.f) {
            const float mnew = fmaxf(m, mt);
            const float corr = fast_exp2(m - mnew);
            m = mnew;
            lsum = ZT_PLANT == 3 ? lsum : lsum * corr;
#pragma unroll
            for (int i = 0; i < NT; ++i) o[i] *= ZT_PLANT == 3 ? 1.f : corr;
        }
        // A key part after the first (KS > 1) can meet a row whose every key so far is masked
        // (its first tile lies past the row, with queries at an offset): the
        // base is still -inf there, and is taken as 0 so that exp2(-inf) = 0.
        const float mb = (KS > 1 && m == -INFINITY) ? 0.f : m;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) s[j][r] = fast_exp2(s[j][r] - mb);
        float ps = s[0][0];  // = 0 + s[0][0]: the weights are >= +0
#pragma unroll
        for (int i = 1; i < 4 * NJ; ++i) ps += s[i / 4][i % 4];
        lsum += ps;

#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            if (k0 + 16 * j >= kend_w) continue;
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                // A operand V^T in the row-owner layout: V[key 16 j + 4 grp + kk][l16 * NT + i].
                float vx[NT];
                lds_run<NT>(vx, Vs + kt + (16 * j + 4 * grp + kk) * LW, l16);
#pragma unroll
                for (int i = 0; i < NT; ++i) o[i] = mfma16(vx[i], s[j][kk], o[i]);
            }
        }
    }

    if constexpr (KS > 1) {
        // Merge the key parts: parts 1.. leave their base, partial sum and
        // output in LDS, part 0 rescales to the larger base and adds them, in
        // part order (a part that saw no visible key has m = -inf and
        // contributes nothing).
        __syncthreads();  // every wave's last reads of the staged tiles
        auto slot = [&](int part) { return smem + (((part - 1) * (NW / KS) + wr) * 64 + lane) * (4 * NT + 2); };
        if (kh > 0) {
            float *mb = slot(kh);
#pragma unroll
            for (int i = 0; i < NT; ++i) *reinterpret_cast<f4 *>(mb + 4 * i) = o[i];
            mb[4 * NT] = m;
            mb[4 * NT + 1] = lsum;
        }
        __syncthreads();
        if (kh == 0) {
#pragma unroll
            for (int part = 1; part < KS; ++part) {
                const float *mb = slot(part);
                const float m2 = mb[4 * NT], l2 = mb[4 * NT + 1];
                const float mm = fmaxf(m, m2);
                const float f1 = m == -INFINITY ? 0.f : fast_exp2(m - mm);
                const float f2 = m2 == -INFINITY ? 0.f : fast_exp2(m2 - mm);
                lsum = lsum * f1 + l2 * f2;
#pragma unroll
                for (int i = 0; i < NT; ++i) o[i] = o[i] * f1 + *reinterpret_cast<const f4 *>(mb + 4 * i) * f2;
                m = mm;
            }
        }
        if (kh != 0) return;  // the merged rows are part 0's to write (no barrier follows in this tile)
    }
    const float l = sum4grp(lsum);
    const float inv = 1.f / l;
    if (a.lse && grp == 0 && my_row < a.T)  // natural log: (m + log2 l) ln 2
        a.lse[((size_t)b * a.T + my_row) * a.H + h] = (m + log2f(l)) * 0.69314718055994531f;
    if (my_row < a.T) {
        float *orow = a.out + (size_t)b * a.T * qld + (size_t)my_row * qld + (size_t)h * a.dim;
#pragma unroll
        for (int r = 0; r < 4; ++r) store_run<NT>(orow, 4 * grp + r, a.dim, vec4, o, r, inv);
    }
}

// Row tile n - 1 - p (latest, heaviest first); with a.pair also row tile p,
// so that every workgroup has the same causal work.
template <int DP, int BK, int NW, bool PF, int KS = 1>
__device__ __forceinline__ void attn_fwd_body(const FwdArgs &a) {
    const int p = (int)blockIdx.x / (a.n_head_blocks * a.B);
    attn_fwd_tile<DP, BK, NW, PF, KS>(a, a.n_row_tiles - 1 - p);
    if (a.pair && p < a.n_row_tiles - 1 - p) {  // workgroup-uniform
        __syncthreads();  // the first tile's last LDS reads before the second's writes
        attn_fwd_tile<DP, BK, NW, PF, KS>(a, p);
    }
}

#define ZT_FWD(DP, BK)                                                                             \
    extern "C" __global__ void __launch_bounds__(256) zt_fwd_d##DP##_k##BK(FwdArgs a) {          \
        attn_fwd_body<DP, BK, 4, false>(a);                                                        \
    }                                                                                              \
    extern "C" __global__ void __launch_bounds__(512) zt_fwd8_d##DP##_k##BK(FwdArgs a) {         \
        attn_fwd_body<DP, BK, 8, false>(a);                                                        \
    }
// Register-prefetched variants (32-key tiles).
#define ZT_FWD_PF(DP)                                                                              \
    extern "C" __global__ void __launch_bounds__(256) zt_fwdp_d##DP##_k32(FwdArgs a) {           \
        attn_fwd_body<DP, 32, 4, true>(a);                                                         \
    }                                                                                              \
    extern "C" __global__ void __launch_bounds__(512, (DP) <= 128 ? 4 : 1) zt_fwd8p_d##DP##_k32(FwdArgs a) { \
        attn_fwd_body<DP, 32, 8, true>(a);                                                         \
    }

// The same eight-wave kernel under its own name for launches that keep the
// scores (s_out set), so that a profile tells the two roles apart.
#define ZT_FWD_PFS(DP)                                                                             \
    extern "C" __global__ void __launch_bounds__(512, 4) zt_fwd8ps_d##DP##_k32(FwdArgs a) {      \
        attn_fwd_body<DP, 32, 8, true>(a);                                                         \
    }

// The key-split variant for heads that share no kv group with another (HW =
// 1) on small grids: eight waves, 4 row blocks x 2 key parts.  (Four key parts
// in sixteen waves measured no better: C2's forward 51.3 us against 54.1 us,
// one 16-head sequence of 2048 rows at d = 64 85.5 against 86.7 us.)
#define ZT_FWD_PFK(DP)                                                                             \
    extern "C" __global__ void __launch_bounds__(512) zt_fwdpk_d##DP##_k32(FwdArgs a) {          \
        attn_fwd_body<DP, 32, 8, true, 2>(a);                                                      \
    }

#if ZT_PLANT == 0
ZT_FWD(32, 32) ZT_FWD(32, 64)
ZT_FWD(64, 32) ZT_FWD(64, 64)
ZT_FWD(96, 32) ZT_FWD(96, 64)
ZT_FWD(128, 32) ZT_FWD(128, 64)
ZT_FWD(160, 32) ZT_FWD(160, 64)
ZT_FWD(192, 32) ZT_FWD(192, 64)
ZT_FWD(224, 32) ZT_FWD(224, 64)
ZT_FWD(256, 32) ZT_FWD(256, 64)
ZT_FWD_PF(32) ZT_FWD_PF(64) ZT_FWD_PF(96) ZT_FWD_PF(128)
ZT_FWD_PF(160) ZT_FWD_PF(192) ZT_FWD_PF(224) ZT_FWD_PF(256)
ZT_FWD_PFS(32) ZT_FWD_PFS(64) ZT_FWD_PFS(96) ZT_FWD_PFS(128)
ZT_FWD_PFK(32) ZT_FWD_PFK(64) ZT_FWD_PFK(96) ZT_FWD_PFK(128)
#else
// A planted-defect build (test-only): the kernels of the negative-control
// shapes, d = 32 (the reference entry points) and d = 128 (the training path).
ZT_FWD_PF(32) ZT_FWD_PF(128) ZT_FWD_PFS(128)
#endif
