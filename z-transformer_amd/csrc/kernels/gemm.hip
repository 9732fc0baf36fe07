// f32 GEMM on FP32 MFMA for the model's dense products (gfx950):
//   zt_gemm_nn: C  = A B      src/tensor.zig:78-106 (tensor.matmul)
//   zt_gemm_tn: C += A^T B    src/autograd.zig:958-972 (weightGrad: w += input^T dout)
//   zt_gemm_nt: C += A B^T    src/autograd.zig:999-1022 (inputGrad: d input += dout w^T)
// All matrices row-major f32.  op(A) is M x K, op(B) is K x N, C is M x N.
//
// Slab kernels: a workgroup of 4 waves computes a BT x BT tile of C (BT = 128,
// or 64 / 32 when the product is too small to fill the device with 128-tiles;
// products smaller still take the split-K kernels further down), each wave
// a quarter as TW x TW tiles of 16 x 16 (TW = BT / 32): up to 16 independent
// accumulation chains of v_mfma_f32_16x16x4_f32.  Each 32-deep k slab of both operands is copied to
// LDS in the orientation it has in memory, with 16-byte loads and stores:
//   * k-contiguous (A as stored, B^T as stored): LDS [index][k], stride 36.
//     Lane group grp owns k in [8 grp, 8 grp + 8) of the slab (the contraction
//     is order-free across k-steps), so one 128-bit read gives a lane's
//     operand for four k-steps of one tile; tile t's local index l16 is
//     16 t + l16 of the wave's 64.
//   * index-contiguous (A^T or B as stored): LDS [k][index], stride BT + 4.
//     Here a lane's TW tiles are the TW consecutive indices TW l16 + t, so
//     one TW-float read gives its operand for all its tiles at one k.
// Either way a k-step group of 4 x TW x TW MFMAs needs four LDS reads per
// operand, and no scattered (transposing) LDS writes are needed.  The next slab
// is prefetched into registers while the current one computes.  Accumulation
// is f32 inside the MFMA; the result differs from the reference's sequential
// f32 sum only in rounding order.
#include "common.h"
#include "args.h"

namespace {

constexpr int BK = 32, NTHR = 256;
constexpr int LKC = BK + 4;  // row stride of a k-contiguous slab

// The 4 floats p[0..3] of a row with `avail` valid elements from p: one
// 16-byte load when vec and all 4 are valid, else guarded scalar loads.
DEVI f4 load4(const float *p, int avail, bool vec) {
    if (vec && avail >= 4) return *reinterpret_cast<const f4 *>(p);
    f4 x = zero4();
    if (avail > 0) x.x = p[0];
    if (avail > 1) x.y = p[1];
    if (avail > 2) x.z = p[2];
    if (avail > 3) x.w = p[3];
    return x;
}

// Workgroup tile BT x BT (128, 64 or 32); each of the 4 waves owns a quarter,
// TW x TW MFMA tiles of 16 x 16.
template <int BT>
struct Tile {
    static constexpr int TW = BT / 32;             // MFMA tiles per wave per dimension
    static constexpr int WT = BT / 2;              // wave tile width
    static constexpr int LIC = BT + 4;             // row stride of an index-contiguous slab
    static constexpr int NCH = BT * BK / 4 / NTHR; // 16-byte chunks per thread per operand
};

// Slab fetch of one operand into registers.  KC: memory rows are the tile
// index (r0.., < rmax), k contiguous (k0.., < kmax).  Otherwise memory rows
// are k and the index is contiguous.
template <int BT, bool KC>
DEVI void fetch(f4 (&pf)[Tile<BT>::NCH], const float *base, int ld, int r0, int rmax, int k0, int kmax, bool vec,
                int tid) {
#pragma unroll
    for (int n = 0; n < Tile<BT>::NCH; ++n) {
        const int e = tid + n * NTHR;
        if constexpr (KC) {
            const int r = r0 + e / (BK / 4), k = k0 + 4 * (e % (BK / 4));
            pf[n] = r < rmax ? load4(base + (size_t)r * ld + k, kmax - k, vec) : zero4();
        } else {
            const int k = k0 + e / (BT / 4), r = r0 + 4 * (e % (BT / 4));
            pf[n] = k < kmax ? load4(base + (size_t)k * ld + r, rmax - r, vec) : zero4();
        }
    }
}

template <int BT, bool KC>
DEVI void put(float *lds, const f4 (&pf)[Tile<BT>::NCH], int tid) {
#pragma unroll
    for (int n = 0; n < Tile<BT>::NCH; ++n) {
        const int e = tid + n * NTHR;
        if constexpr (KC)
            *reinterpret_cast<f4 *>(lds + (e / (BK / 4)) * LKC + 4 * (e % (BK / 4))) = pf[n];
        else
            *reinterpret_cast<f4 *>(lds + (e / (BT / 4)) * Tile<BT>::LIC + 4 * (e % (BT / 4))) = pf[n];
    }
}

// A lane's operand block x[t][c] for its tiles t < TW and k-steps c = 0..3 of
// half h of the slab; w0 = the wave's first index.  KC: one 128-bit read per
// tile.  Otherwise the lane's tiles are the TW consecutive indices TW l16 + t:
// one TW-float read per k-step.
template <int BT, bool KC>
DEVI void operand(f4 (&x)[Tile<BT>::TW], const float *lds, int w0, int l16, int grp, int h) {
    constexpr int TW = Tile<BT>::TW;
    if constexpr (KC) {
#pragma unroll
        for (int t = 0; t < TW; ++t)
            x[t] = *reinterpret_cast<const f4 *>(lds + (w0 + 16 * t + l16) * LKC + 8 * grp + 4 * h);
    } else {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float *p = lds + (8 * grp + 4 * h + c) * Tile<BT>::LIC + w0 + TW * l16;
            if constexpr (TW == 4) {
                const f4 y = *reinterpret_cast<const f4 *>(p);
#pragma unroll
                for (int t = 0; t < 4; ++t) x[t][c] = y[t];
            } else if constexpr (TW == 2) {
                const f2 y = *reinterpret_cast<const f2 *>(p);
                x[0][c] = y.x; x[1][c] = y.y;
            } else {
                x[0][c] = *p;
            }
        }
    }
}

// Index within the wave's tile of MFMA tile t's local row/column j.
template <int TW, bool KC>
DEVI int local_index(int t, int j) { return KC ? 16 * t + j : TW * j + t; }

// Offsets (floats, from the operand's base) of a thread's slab chunks when
// every chunk is inside the matrix: fixed for the kernel apart from the
// slab's k0, which moves the base (a scalar) by k0 (KC) or k0 rows (else).
template <int BT, bool KC>
DEVI void chunk_offsets(unsigned (&off)[Tile<BT>::NCH], int ld, int r0, int tid) {
#pragma unroll
    for (int n = 0; n < Tile<BT>::NCH; ++n) {
        const int e = tid + n * NTHR;
        off[n] = KC ? (unsigned)(r0 + e / (BK / 4)) * (unsigned)ld + 4u * (unsigned)(e % (BK / 4))
                    : (unsigned)(e / (BT / 4)) * (unsigned)ld + (unsigned)r0 + 4u * (unsigned)(e % (BT / 4));
    }
}

// A_KC: A stored M x K (else K x M).  B_KC: B stored N x K (else K x N).
// FULL: M and N multiples of BT, K of BK, 16-byte rows: every slab chunk is
// inside its matrix, so the loads are unconditional 16-byte loads from a
// scalar slab base plus a fixed per-thread offset (no bounds arithmetic or
// branches per chunk), and C is stored without bounds checks.
template <int BT, bool A_KC, bool B_KC, bool FULL>
DEVI void gemm_tile(const GemmArgs &g) {
    using TL = Tile<BT>;
    constexpr int TW = TL::TW, NCH = TL::NCH;
    __shared__ __attribute__((aligned(16))) float As[A_KC ? BT * LKC : BK * TL::LIC];
    __shared__ __attribute__((aligned(16))) float Bs[B_KC ? BT * LKC : BK * TL::LIC];
    const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, grp = lane >> 4, w = tid >> 6;
    const int wm = TL::WT * (w >> 1), wn = TL::WT * (w & 1);
    const int tiles_n = (g.N + BT - 1) / BT;
    const int m0 = (int)(blockIdx.x / tiles_n) * BT, n0 = (int)(blockIdx.x % tiles_n) * BT;

    f4 acc[TW][TW];
#pragma unroll
    for (int i = 0; i < TW; ++i)
#pragma unroll
        for (int j = 0; j < TW; ++j) acc[i][j] = zero4();

    f4 pa[NCH], pb[NCH];
    unsigned oa[FULL ? NCH : 1], ob[FULL ? NCH : 1];
    auto fetch_full = [&](f4 (&pf)[NCH], const unsigned (&off)[FULL ? NCH : 1], const float *base) {
#pragma unroll
        for (int n = 0; n < NCH; ++n) pf[n] = *reinterpret_cast<const f4 *>(base + off[n]);
    };
    // The slab base at k0: k0 columns on (k contiguous) or k0 rows down.
    auto slab = [](const float *p, int ld, bool kc, int k0) { return kc ? p + k0 : p + (size_t)k0 * ld; };
    if constexpr (FULL) {
        chunk_offsets<BT, A_KC>(oa, g.lda, m0, tid);
        chunk_offsets<BT, B_KC>(ob, g.ldb, n0, tid);
        fetch_full(pa, oa, g.a);
        fetch_full(pb, ob, g.b);
    } else {
        fetch<BT, A_KC>(pa, g.a, g.lda, m0, g.M, 0, g.K, g.vec_a, tid);
        fetch<BT, B_KC>(pb, g.b, g.ldb, n0, g.N, 0, g.K, g.vec_b, tid);
    }
    for (int k0 = 0; k0 < g.K; k0 += BK) {
        __syncthreads();
        put<BT, A_KC>(As, pa, tid);
        put<BT, B_KC>(Bs, pb, tid);
        __syncthreads();
        if (k0 + BK < g.K) {
            if constexpr (FULL) {
                fetch_full(pa, oa, slab(g.a, g.lda, A_KC, k0 + BK));
                fetch_full(pb, ob, slab(g.b, g.ldb, B_KC, k0 + BK));
            } else {
                fetch<BT, A_KC>(pa, g.a, g.lda, m0, g.M, k0 + BK, g.K, g.vec_a, tid);
                fetch<BT, B_KC>(pb, g.b, g.ldb, n0, g.N, k0 + BK, g.K, g.vec_b, tid);
            }
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            f4 av[TW], bv[TW];
            operand<BT, A_KC>(av, As, wm, l16, grp, h);
            operand<BT, B_KC>(bv, Bs, wn, l16, grp, h);
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int i = 0; i < TW; ++i)
#pragma unroll
                    for (int j = 0; j < TW; ++j) acc[i][j] = mfma16(av[i][c], bv[j][c], acc[i][j]);
        }
    }

    // acc[i][j][r] = C[m0 + wm + local_index(i, 4 grp + r)][n0 + wn + local_index(j, l16)]
#pragma unroll
    for (int i = 0; i < TW; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = m0 + wm + local_index<TW, A_KC>(i, 4 * grp + r);
            if (!FULL && m >= g.M) continue;
            float *crow = g.c + (size_t)m * g.ldc;
            if constexpr (!B_KC && TW == 4) {  // the lane's four columns are consecutive
                const int n = n0 + wn + 4 * l16;
                f4 v;
#pragma unroll
                for (int j = 0; j < 4; ++j) v[j] = acc[i][j][r];
                if (FULL || (g.vec_c && n + 3 < g.N)) {
                    f4 *p = reinterpret_cast<f4 *>(crow + n);
                    *p = g.accumulate ? *p + v : v;
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (n + j < g.N) crow[n + j] = g.accumulate ? crow[n + j] + v[j] : v[j];
                }
            } else {
#pragma unroll
                for (int j = 0; j < TW; ++j) {
                    const int n = n0 + wn + local_index<TW, B_KC>(j, l16);
                    if (FULL || n < g.N) crow[n] = g.accumulate ? crow[n] + acc[i][j][r] : acc[i][j][r];
                }
            }
        }
}
template <int BT, bool A_KC, bool B_KC>
DEVI void gemm_body(const GemmArgs &g) {
    // Workgroup-uniform: the whole product is in full tiles (vec_c as well,
    // so the C rows take 16-byte stores), and a k-contiguous operand's chunk
    // offsets (up to M lda or N ldb floats) fit the 32-bit offsets.
    constexpr unsigned long long kOff = 1ull << 32;
    const bool full = g.vec_a && g.vec_b && g.vec_c && g.M % BT == 0 && g.N % BT == 0 && g.K % BK == 0 &&
                      (!A_KC || (unsigned long long)g.M * (unsigned)g.lda < kOff) &&
                      (!B_KC || (unsigned long long)g.N * (unsigned)g.ldb < kOff);
    if (full) gemm_tile<BT, A_KC, B_KC, true>(g);
    else gemm_tile<BT, A_KC, B_KC, false>(g);
}

// Split-K variant for products too small to fill the device with slab tiles
// (the model's own: 256 x 512 x 128 and the like).  There the slab kernels'
// serial walk over K, a global-load round trip and two barriers per 32-deep
// slab on a handful of workgroups, sets the time, not the MFMAs.
//
// A workgroup of NW waves (NW = blockDim.x / 64: 4, 8 or 16) owns a
// 16 TW x 16 TW tile of C.  The waves split K into 16-deep blocks taken
// round-robin (wave w: blocks w, w + NW, ...); each wave loads its blocks'
// operands straight from global memory into MFMA operand registers (no LDS
// staging, no barrier), the next block's loads issued before the current
// block's MFMAs.  Lane group grp holds k = 16 kb + 4 grp + c at k-step c, as
// the slab kernels do.  The NW partial tiles are then summed through LDS in
// wave order: the result does not depend on timing, and needs neither atomics
// nor a workspace.
constexpr int SK_MAXW = 16;

// MFMA operand of index r (this lane's row of op(X)) at k .. k+3 (this lane's
// k-steps), zero past rmax / kmax.  KC: X stored index-major, k contiguous.
template <bool KC>
DEVI f4 sk_operand(const float *base, int ld, int r, int rmax, int k, int kmax, bool vec) {
    f4 x = zero4();
    if (r >= rmax) return x;
    if constexpr (KC) {
        x = load4(base + (size_t)r * ld + k, kmax - k, vec);
    } else {
#pragma unroll
        for (int c = 0; c < 4; ++c)
            if (k + c < kmax) x[c] = base[(size_t)(k + c) * ld + r];
    }
    return x;
}

template <int TW, bool A_KC, bool B_KC>
DEVI void gemm_sk_body(const GemmArgs &g) {
    constexpr int E = TW * TW * 256;  // floats of the workgroup's tile
    __shared__ __attribute__((aligned(16))) float red[SK_MAXW * E];
    const int tid = threadIdx.x, lane = tid & 63, l16 = lane & 15, grp = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6), nw = (int)(blockDim.x >> 6);
    const int tiles_n = (g.N + 16 * TW - 1) / (16 * TW);
    const int m0 = (int)(blockIdx.x / tiles_n) * 16 * TW, n0 = (int)(blockIdx.x % tiles_n) * 16 * TW;
    const int nkb = (g.K + 15) >> 4;

    f4 acc[TW][TW];
#pragma unroll
    for (int i = 0; i < TW; ++i)
#pragma unroll
        for (int j = 0; j < TW; ++j) acc[i][j] = zero4();

    auto load = [&](f4 (&a)[TW], f4 (&b)[TW], int kb) {
        const int k = 16 * kb + 4 * grp;
#pragma unroll
        for (int t = 0; t < TW; ++t) {
            a[t] = sk_operand<A_KC>(g.a, g.lda, m0 + 16 * t + l16, g.M, k, g.K, g.vec_a);
            b[t] = sk_operand<B_KC>(g.b, g.ldb, n0 + 16 * t + l16, g.N, k, g.K, g.vec_b);
        }
    };
    auto mma = [&](const f4 (&a)[TW], const f4 (&b)[TW]) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int i = 0; i < TW; ++i)
#pragma unroll
                for (int j = 0; j < TW; ++j) acc[i][j] = mfma16(a[i][c], b[j][c], acc[i][j]);
    };

    // Two register sets: the block after next loads while a block computes.
    f4 a0[TW], b0[TW], a1[TW], b1[TW];
    if (w < nkb) load(a0, b0, w);
    for (int kb = w; kb < nkb; kb += 2 * nw) {  // wave-uniform
        if (kb + nw < nkb) load(a1, b1, kb + nw);
        mma(a0, b0);
        if (kb + nw >= nkb) break;
        if (kb + 2 * nw < nkb) load(a0, b0, kb + 2 * nw);
        mma(a1, b1);
    }

    // acc[i][j][r] = partial C[m0 + 16 i + 4 grp + r][n0 + 16 j + l16], stored
    // at ((i TW + j) 4 + r) 64 + lane of the wave's slot.
    float *const mine = red + w * E;
#pragma unroll
    for (int i = 0; i < TW; ++i)
#pragma unroll
        for (int j = 0; j < TW; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) mine[((i * TW + j) * 4 + r) * 64 + lane] = acc[i][j][r];
    __syncthreads();
    for (int e = tid; e < E; e += (int)blockDim.x) {
        float s = red[e];
        for (int ww = 1; ww < nw; ++ww) s += red[ww * E + e];
        const int ln = e & 63, r = (e >> 6) & 3, ij = e >> 8;
        const int m = m0 + 16 * (ij / TW) + 4 * (ln >> 4) + r, n = n0 + 16 * (ij % TW) + (ln & 15);
        if (m < g.M && n < g.N) {
            float *p = g.c + (size_t)m * g.ldc + n;
            *p = g.accumulate ? *p + s : s;
        }
    }
}

// dq from a stored dS (the training backward's workspace path):
//   dq[b, t, h, :] = scale * sum_{s <= t} dS[b, h, t, s] k[b, s, h / group, :]
// A GEMM per (sequence, head): A = dS, B = k rows (index-contiguous: the head
// dimension), C = dq rows; the reduction stops at the row tile's last query.
// dS arrives in 16 x 16 tiles in lane order (the dk/dv kernel's store): a
// 16-byte chunk of a tile is 4 consecutive queries at one key, which is the
// index-contiguous orientation of A, so slabs are staged with 16-byte loads and
// stores; tiles above the diagonal (never written) and rows past T read as 0.
// Grid: row-tile pairs, then (sequence, head), then column tiles.
// The dS and K slabs: one allocation per tile size, shared by the aligned and
// unaligned instantiations.
template <int BT, int KSP>
DEVI float *dq_ds_slabs() {
    __shared__ __attribute__((aligned(16))) float slabs[KSP * 2 * BK * Tile<BT>::LIC];
    return slabs;
}
// KSP key parts (KSP = 2: eight waves, for grids that give a workgroup of four
// per CU): part kp of the workgroup's threads -- four waves, a whole tile --
// takes key slabs kp, kp + KSP, ... into its own LDS slabs, and the parts'
// tiles are added through LDS in part order at the end.
template <int BT, bool VEC, int KSP = 1>
DEVI void dq_ds_tile(const DqDsArgs &g, const int tm, const int tn, const int bh) {
    using TL = Tile<BT>;
    constexpr int TW = TL::TW, NCH = TL::NCH;
    static_assert(KSP == 1 || VEC, "the key split takes the unconditional loads");
    const int kp = KSP > 1 ? __builtin_amdgcn_readfirstlane((int)threadIdx.x / NTHR) : 0;
    float *const As = dq_ds_slabs<BT, KSP>() + kp * 2 * BK * TL::LIC, *const Bs = As + BK * TL::LIC;
    const int tid = (int)threadIdx.x % NTHR, lane = tid & 63, l16 = lane & 15, grp = lane >> 4;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = TL::WT * (w >> 1), wn = TL::WT * (w & 1);
    const int b = bh / g.H, h = bh % g.H, kvh = h / (g.H / g.Hkv);
    const int m0 = tm * BT, n0 = tn * BT;
    const size_t qld = (size_t)g.H * g.dim, kld = (size_t)g.Hkv * g.dim;
    const int nt = (g.T + 15) >> 4;
    const float *A = g.ds + (size_t)bh * zt_tri_count(nt) * 256;
    const float *Bm = g.k + (size_t)b * g.T * kld + (size_t)kvh * g.dim;
    float *C = g.dq + (size_t)b * g.T * qld + (size_t)h * g.dim;
    const int kend = min(g.T, m0 + BT);

    f4 acc[TW][TW];
#pragma unroll
    for (int i = 0; i < TW; ++i)
#pragma unroll
        for (int j = 0; j < TW; ++j) acc[i][j] = zero4();

    // A slab: keys k0..k0+31 x queries m0..m0+BT-1 = (BT/16) x 2 tiles; chunk e
    // is (tile, lane-chunk); put() stores it at [key][query .. query+3].
    f4 pa[NCH], pb[NCH];
    // With VEC (16-byte k rows) every load is unconditional and in bounds: a
    // dS tile outside the causal triangle or the grid loads a written one and
    // is zeroed by a select, and key rows past kend load row kend - 1 (met by
    // those zero tiles) and columns past dim the row's last four floats
    // (landing in dq columns never stored).
    auto fetch_a = [&](int k0) {
#pragma unroll
        for (int n = 0; n < NCH; ++n) {
            const int e = tid + n * NTHR;
            const int tile = e >> 6, c = e & 63;         // 64 chunks per tile
            const int tb = (m0 >> 4) + tile % (BT / 16), sb = (k0 >> 4) + tile / (BT / 16);
            const bool ok = sb <= tb && tb < nt;
            if constexpr (VEC) {  // read once: nontemporal
                const int tc = min(tb, nt - 1), sc = min(sb, tc);
                const f4 x = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(A + zt_tri_index(tc, sc) * 256) + c);
                pa[n] = ok ? x : zero4();
            } else {
                f4 x = zero4();
                if (ok) x = __builtin_nontemporal_load(reinterpret_cast<const f4 *>(A + zt_tri_index(tb, sb) * 256) + c);
                pa[n] = x;
            }
        }
    };
    auto fetch_b = [&](int k0) {
        if constexpr (VEC) {
#pragma unroll
            for (int n = 0; n < NCH; ++n) {
                const int e = tid + n * NTHR;
                const int k = min(k0 + e / (BT / 4), kend - 1), r = min(n0 + 4 * (e % (BT / 4)), g.dim - 4);
                pb[n] = *reinterpret_cast<const f4 *>(Bm + (size_t)k * kld + r);
            }
        } else {
            fetch<BT, false>(pb, Bm, (int)kld, n0, g.dim, k0, kend, false, tid);
        }
    };
    auto put_a = [&]() {
#pragma unroll
        for (int n = 0; n < NCH; ++n) {
            const int e = tid + n * NTHR;
            const int tile = e >> 6, c = e & 63;
            const int tl = 16 * (tile % (BT / 16)) + 4 * (c >> 4), sl = 16 * (tile / (BT / 16)) + (c & 15);
            *reinterpret_cast<f4 *>(As + sl * TL::LIC + tl) = pa[n];
        }
    };
    // Step ks covers slabs ks .. ks + KSP - 1, this part's being ks + kp; a
    // part without a slab in the last step fetches the last one again and
    // computes nothing (every part meets every barrier).
    const int last = ((kend - 1) / BK) * BK;
    fetch_a(min(kp * BK, last));
    fetch_b(min(kp * BK, last));
    for (int ks = 0; ks < kend; ks += KSP * BK) {
        const int k0 = ks + kp * BK;
        __syncthreads();
        put_a();
        put<BT, false>(Bs, pb, tid);
        __syncthreads();
        // The next slab (the last one fetches itself again, unused): dS
        // chunks now, K chunks between the two halves' products.
        const int kn = k0 + KSP * BK < kend ? k0 + KSP * BK : min(k0, last);
        if (VEC || k0 + BK < kend) fetch_a(kn);
        if (KSP > 1 && k0 >= kend) {  // wave-uniform: this part has no slab in this step
            fetch_b(kn);
            continue;
        }
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            if (hh == 1 && (VEC || k0 + BK < kend)) fetch_b(kn);
            f4 av[TW], bv[TW];
            operand<BT, false>(av, As, wm, l16, grp, hh);
            operand<BT, false>(bv, Bs, wn, l16, grp, hh);
#pragma unroll
            for (int c = 0; c < 4; ++c)
#pragma unroll
                for (int i = 0; i < TW; ++i)
#pragma unroll
                    for (int j = 0; j < TW; ++j) acc[i][j] = mfma16(av[i][c], bv[j][c], acc[i][j]);
        }
    }
    if constexpr (KSP > 1) {
        // The parts' tiles, added in part order by part 0 (which stores them).
        static_assert((KSP - 1) * NTHR * TW * TW * 4 <= KSP * 2 * BK * TL::LIC, "merge buffer");
        f4 *const red = reinterpret_cast<f4 *>(dq_ds_slabs<BT, KSP>());
        __syncthreads();  // every part's last operand reads
        if (kp > 0) {
#pragma unroll
            for (int i = 0; i < TW; ++i)
#pragma unroll
                for (int j = 0; j < TW; ++j) red[(((kp - 1) * TW + i) * TW + j) * NTHR + tid] = acc[i][j];
        }
        __syncthreads();
        if (kp > 0) return;  // no barrier follows in this tile
#pragma unroll
        for (int q = 1; q < KSP; ++q)
#pragma unroll
            for (int i = 0; i < TW; ++i)
#pragma unroll
                for (int j = 0; j < TW; ++j) acc[i][j] += red[(((q - 1) * TW + i) * TW + j) * NTHR + tid];
    }

#pragma unroll
    for (int i = 0; i < TW; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = m0 + wm + local_index<TW, false>(i, 4 * grp + r);
            if (t >= g.T) continue;
            float *crow = C + (size_t)t * qld;
#pragma unroll
            for (int j = 0; j < TW; ++j) {
                const int n = n0 + wn + local_index<TW, false>(j, l16);
                if (n < g.dim) crow[n] = ZT_PLANT == 16 ? acc[i][j][r] : acc[i][j][r] * g.scale;
            }
        }
}

// A workgroup takes row tiles tiles_m - 1 - p and p one after the other, so
// every workgroup has the same causal work (C3: 0.64 -> 0.58 ms against one
// row tile per workgroup, heaviest first).
template <int BT, int KSP = 1>
DEVI void dq_ds_body(const DqDsArgs &g) {
    int rem = (int)blockIdx.x;
    const int tn = rem % g.tiles_n;
    rem /= g.tiles_n;
    const int bh = rem % (g.B * g.H);
    const int p = rem / (g.B * g.H);
    if (KSP > 1 || g.vec) {  // (the host takes the key-split kernels only with vec)
        dq_ds_tile<BT, true, KSP>(g, g.tiles_m - 1 - p, tn, bh);
        if (p < g.tiles_m - 1 - p) {  // workgroup-uniform
            __syncthreads();  // the first tile's last LDS reads before the second's writes
            dq_ds_tile<BT, true, KSP>(g, p, tn, bh);
        }
    } else {
        dq_ds_tile<BT, false>(g, g.tiles_m - 1 - p, tn, bh);
        if (p < g.tiles_m - 1 - p) {
            __syncthreads();
            dq_ds_tile<BT, false>(g, p, tn, bh);
        }
    }
}

}  // namespace

// Kernel names: zt_gemm_<op>_<tile>.
#define ZT_GEMM(BT)                                                                                \
    extern "C" __global__ void __launch_bounds__(256) zt_gemm_nn_##BT(GemmArgs g) { gemm_body<BT, true, false>(g); } \
    extern "C" __global__ void __launch_bounds__(256) zt_gemm_tn_##BT(GemmArgs g) { gemm_body<BT, false, false>(g); } \
    extern "C" __global__ void __launch_bounds__(256) zt_gemm_nt_##BT(GemmArgs g) { gemm_body<BT, true, true>(g); }

ZT_GEMM(128)
ZT_GEMM(64)
ZT_GEMM(32)

// Split-K kernels: zt_gemm_<op>_sk<16 TW>, 64 NW threads (NW = 4, 8 or 16).
#define ZT_GEMM_SK(TW, BT)                                                                               \
    extern "C" __global__ void __launch_bounds__(1024) zt_gemm_nn_sk##BT(GemmArgs g) { gemm_sk_body<TW, true, false>(g); } \
    extern "C" __global__ void __launch_bounds__(1024) zt_gemm_tn_sk##BT(GemmArgs g) { gemm_sk_body<TW, false, false>(g); } \
    extern "C" __global__ void __launch_bounds__(1024) zt_gemm_nt_sk##BT(GemmArgs g) { gemm_sk_body<TW, true, true>(g); }

ZT_GEMM_SK(1, 16)
ZT_GEMM_SK(2, 32)

extern "C" __global__ void __launch_bounds__(256) zt_gemm_dqds_128(DqDsArgs g) { dq_ds_body<128>(g); }
extern "C" __global__ void __launch_bounds__(256) zt_gemm_dqds_64(DqDsArgs g) { dq_ds_body<64>(g); }
// Two key parts, eight waves (grids of at most one four-wave workgroup per CU).
extern "C" __global__ void __launch_bounds__(512) zt_gemm_dqds2_64(DqDsArgs g) { dq_ds_body<64, 2>(g); }
extern "C" __global__ void __launch_bounds__(512) zt_gemm_dqds2_128(DqDsArgs g) { dq_ds_body<128, 2>(g); }
