// Device-side helpers shared by the gfx950 kernels.
//
// Conventions used by every attention kernel in this directory:
//   * One wavefront is 64 lanes.  lane = threadIdx.x & 63, l16 = lane & 15,
//     grp = lane >> 4 (0..3).
//   * FP32 matrix-core op: v_mfma_f32_16x16x4_f32, D[16x16] += A[16x4] B[4x16].
//       A operand: lane holds A[i = l16][k = grp]
//       B operand: lane holds B[k = grp][j = l16]
//       C/D:       lane holds D[i = 4*grp + r][j = l16], r = 0..3 (one float4)
//   * A contraction over the head dimension d is split so that lane group grp
//     owns d in [grp*DP/4, (grp+1)*DP/4); k-step kk uses d = grp*DP/4 + kk.  A
//     sum is order-free across k-steps, so each lane then reads DP/4
//     contiguous floats of a row (128-bit loads) instead of a strided column.
//   * Products whose output rows run over the head dimension (O^T, dq^T, dK^T,
//     dV^T) use the "row-owner" layout: with C = 4 floats when NT = DP/16 is a
//     multiple of 4 (else C = 2), output row i (0..15) of column tile it
//     (0..NT-1) is d = (it / C) * 16C + C i + it % C.  Row i thus owns the C-float
//     chunk i of every 16C-wide column block, so the A operand a lane needs for
//     one k-step -- row i = l16 of every tile -- is NT/C chunks of one row-major
//     LDS row (128- or 64-bit reads, lds_run) with consecutive lanes on
//     consecutive chunks (no bank conflicts), and accumulator row 4*grp + r
//     holds whole C-float chunks of one output row (store_run).
//   * Scores are kept transposed (keys on the M axis, queries on the N axis):
//     the C layout of S^T (lane = query column, 4 key rows per register group)
//     is then exactly the B-operand layout the P.V product needs, with key
//     4*grp + kk on k-step kk.  P never leaves registers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// Planted defects.  ZT_PLANT selects one of the defects below for the
// test-only code objects that the negative-control tests load (built by
// tests/planted/build.py, each into its own test library); libzt_attn.so is
// built without it, so every `if constexpr (ZT_PLANT == n)` folds away and
// its kernels carry no trace of them.  Each is a defect a real kernel of
// this kind can ship with:
//   1  forward: causal mask dropped (a query sees the later keys of its tile)
//   2  forward: every query head reads kv head 0 (GQA collapsed)
//   3  forward: the online softmax's running-max rescale skipped
//   4  forward: the 1/sqrt(d) scale dropped
//   5  training forward: the score tiles it keeps for the backward are stored
//      without the log2(e)/sqrt(d) scale (O and lse stay right)
//   11 backward: causal mask dropped in the dq and dk/dv kernels
//   12 backward: K and V read from kv head 0 for every kv group
//   13 backward: the softmax Jacobian dropped (dS = P, so dv stays right)
//   14 backward: the 1/sqrt(d) scale dropped (scores, dq and dk)
//   15 score-reading dk/dv: a stage's two dS sub-tiles stored in each other's
//      slots (dk and dv stay right, the dq product reads the wrong tiles)
//   16 dq-from-dS product: the 1/sqrt(d) scale dropped (dq = sqrt(d) x right)
//   17 decode combine: the last chunk of a split sequence left out of the merge
//   21 RMSNorm: the first weight element moved by 1e-3
//   22 RMSNorm: the mean of x instead of the mean of its squares
//   23 RMSNorm: the weight read from x (the wrong tensor at the right index)
#ifndef ZT_PLANT
#define ZT_PLANT 0
#endif

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));

#define DEVI __device__ __forceinline__

constexpr float kLog2e = 1.4426950408889634f;

DEVI f4 mfma16(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

DEVI int lane_id() { return threadIdx.x & 63; }

// 2^x on the hardware's v_exp_f32, without the library's rescaling of
// results below 2^-126: softmax weights that small are negligible next to a
// row sum of at least 1.  2^-inf = 0.
DEVI float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

DEVI float wave_xor(float v, int mask) { return __shfl_xor(v, mask, 64); }

// Lane l's value and lane l ^ 16's (l ^ 32's), in some order, from gfx950's
// row-swap instructions: v_permlane16_swap with both operands v exchanges the
// odd 16-lane rows of the first copy with the even rows of the second, so each
// copy then holds, per lane, one of the pair {v[l], v[l ^ 16]} and the other
// copy the other; v_permlane32_swap does the same for the two 32-lane halves.
// VALU only: no LDS round trip as a cross-row shuffle takes.
DEVI void pair16(float v, float &a, float &b) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
}
DEVI void pair32(float v, float &a, float &b) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    a = __uint_as_float(r[0]);
    b = __uint_as_float(r[1]);
}

// Maxima on v_max_f32 / v_max3_f32 as they stand.  fmaxf first quiets every
// operand the compiler cannot show to be quiet, one more v_max_f32 x, x, x per
// MFMA result or lane-swapped copy; the operands here are those and never
// signalling NaNs, for which the two agree (a quiet NaN operand yields the
// other operand, in the hardware's IEEE mode as in fmaxf).
DEVI float vmax(float a, float b) {
    float r;
    asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
DEVI float vmax3(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}
// Maximum of the N values x[0..N).
template <int N>
DEVI float vmax_n(const float (&x)[N]) {
    static_assert(N >= 2, "two values at least");
    float m = vmax(x[0], x[1]);
    int i = 2;
#pragma unroll
    for (; i + 1 < N; i += 2) m = vmax3(m, x[i], x[i + 1]);
    if (i < N) m = vmax(m, x[i]);
    return m;
}

DEVI float max4grp(float v) {  // max over the four lane groups sharing l16
    float a, b;
    pair16(v, a, b);
    pair32(vmax(a, b), a, b);
    return vmax(a, b);
}
// Sum over the four lane groups sharing l16 (each step adds one pair, and a
// two-operand f32 add does not depend on operand order, so all four agree).
DEVI float sum4grp(float v) {
    float a, b;
    pair16(v, a, b);
    pair32(a + b, a, b);
    return a + b;
}

DEVI f4 zero4() { return f4{0.f, 0.f, 0.f, 0.f}; }

// Loads `n` floats (n a multiple of 4) of a row starting at column c0 into
// dst, zero for columns >= dim.  `vec4` says rows are 16-byte aligned and dim
// is a multiple of 4; otherwise rows are only 8-byte aligned (dim even) and
// float2 loads are used.  Wave-uniform branch.
template <int N>
DEVI void load_row_seg(float *dst, const float *row, int c0, int dim, bool vec4, bool valid, float mul) {
    if (vec4) {
#pragma unroll
        for (int i = 0; i < N; i += 4) {
            f4 x = zero4();
            if (valid && c0 + i < dim) x = *reinterpret_cast<const f4 *>(row + c0 + i);
            dst[i] = x.x * mul; dst[i + 1] = x.y * mul; dst[i + 2] = x.z * mul; dst[i + 3] = x.w * mul;
        }
    } else {
#pragma unroll
        for (int i = 0; i < N; i += 2) {
            f2 x = f2{0.f, 0.f};
            if (valid && c0 + i < dim) x = *reinterpret_cast<const f2 *>(row + c0 + i);
            dst[i] = x.x * mul; dst[i + 1] = x.y * mul;
        }
    }
}

// Stores float4 `x` at row[c0..c0+3], columns >= dim dropped.
DEVI void store4(float *row, int c0, int dim, bool vec4, f4 x) {
    if (vec4) {
        if (c0 < dim) *reinterpret_cast<f4 *>(row + c0) = x;
    } else {
        if (c0 < dim) *reinterpret_cast<f2 *>(row + c0) = f2{x.x, x.y};
        if (c0 + 2 < dim) *reinterpret_cast<f2 *>(row + c0 + 2) = f2{x.z, x.w};
    }
}

// Row-owner chunk width (floats) for NT column tiles.
template <int NT>
constexpr int ro_chunk() { return NT % 4 == 0 ? 4 : 2; }

// Reads the row-owner A operand of row rho from one LDS row: x[it] = row[d(rho, it)].
// Rows must be 4C-byte aligned.
template <int NT>
DEVI void lds_run(float (&x)[NT], const float *row, int rho) {
    constexpr int C = ro_chunk<NT>();
#pragma unroll
    for (int c = 0; c < NT / C; ++c) {
        const float *p = row + 16 * C * c + C * rho;
        if constexpr (C == 4) {
            const f4 v = *reinterpret_cast<const f4 *>(p);
            x[4 * c] = v.x; x[4 * c + 1] = v.y; x[4 * c + 2] = v.z; x[4 * c + 3] = v.w;
        } else {
            const f2 v = *reinterpret_cast<const f2 *>(p);
            x[2 * c] = v.x; x[2 * c + 1] = v.y;
        }
    }
}

// Stores accumulator row r (output row rho = 4 grp + r) of row-owner
// accumulators, acc[it][r] * mul, to its columns of `row`; columns >= dim are
// dropped.  128-bit stores for 4-float chunks on 16-byte aligned rows (vec4),
// else 64-bit stores (dim and chunk starts are even, so a pair never straddles dim).
template <int NT>
DEVI void store_run(float *row, int rho, int dim, bool vec4, const f4 (&acc)[NT], int r, float mul) {
    constexpr int C = ro_chunk<NT>();
#pragma unroll
    for (int c = 0; c < NT / C; ++c) {
        const int col = 16 * C * c + C * rho;
        if constexpr (C == 4) {
            const f4 v = f4{acc[4 * c][r], acc[4 * c + 1][r], acc[4 * c + 2][r], acc[4 * c + 3][r]} * mul;
            if (vec4) {
                if (col < dim) *reinterpret_cast<f4 *>(row + col) = v;
            } else {
                if (col < dim) *reinterpret_cast<f2 *>(row + col) = f2{v.x, v.y};
                if (col + 2 < dim) *reinterpret_cast<f2 *>(row + col + 2) = f2{v.z, v.w};
            }
        } else {
            if (col < dim) *reinterpret_cast<f2 *>(row + col) = f2{acc[2 * c][r], acc[2 * c + 1][r]} * mul;
        }
    }
}

// Cooperative copy of `rows` rows x DP columns (global row stride `ld`
// floats) into LDS rows of stride LDSW floats.  Rows >= nvalid and columns
// >= dim are written as zero.  NT threads take part.
template <int DP, int LDSW, int NT>
DEVI void stage_rows(float *lds, const float *g, size_t ld, int rows, int nvalid, int dim, bool vec4,
                     int tid) {
    if (vec4) {
        constexpr int CPR = DP / 4;  // float4 chunks per row
        for (int e = tid; e < rows * CPR; e += NT) {
            const int r = e / CPR, c = (e % CPR) * 4;
            f4 x = zero4();
            if (r < nvalid && c < dim) x = *reinterpret_cast<const f4 *>(g + (size_t)r * ld + c);
            *reinterpret_cast<f4 *>(lds + r * LDSW + c) = x;
        }
    } else {
        constexpr int CPR = DP / 2;
        for (int e = tid; e < rows * CPR; e += NT) {
            const int r = e / CPR, c = (e % CPR) * 2;
            f2 x = f2{0.f, 0.f};
            if (r < nvalid && c < dim) x = *reinterpret_cast<const f2 *>(g + (size_t)r * ld + c);
            *reinterpret_cast<f2 *>(lds + r * LDSW + c) = x;
        }
    }
}

// Asynchronous 16-byte global -> LDS copy (gfx950 global_load_lds_dwordx4): the
// 64 lanes' 16 bytes land contiguously at lds_base + 16 * lane.  lds_base must
// be the same for the whole wave.  Completion is awaited with wait_dma().
DEVI void dma16(const float *g, float *lds_base) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void *)lds_base, 16, 0, 0);
}
DEVI void wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// LDS tiles filled by dma16 have no row padding; instead the 16-byte chunk c of
// row r is stored at chunk position c ^ (r & M), M = 15 when a row has a
// multiple of 16 chunks (DP a multiple of 64), else 7.  With 16 rows read at one
// column (MFMA A operand) the XOR puts them on 16 distinct 4-bank groups, and
// with the 4 rows 4 apart a transposed read visits, their 4-chunk runs on 4
// distinct groups: both conflict-free on 64 banks, as a +4-float pad is.  The
// XOR stays inside an aligned group of M+1 chunks, so a row maps onto itself.
template <int CPR>
DEVI int swz(int chunk, int row) { return chunk ^ (row & (CPR % 16 == 0 ? 15 : 7)); }

// The row-owner A operand of row rho from row r of a swizzled unpadded tile (see swz).
template <int NT, int CPR>
DEVI void lds_run_swz(float (&x)[NT], const float *tile, int r, int rho) {
    constexpr int C = ro_chunk<NT>();
    const float *rowp = tile + r * CPR * 4;
#pragma unroll
    for (int c = 0; c < NT / C; ++c) {
        const int col = 16 * C * c + C * rho;  // a C-float chunk never leaves its 16-byte chunk
        const float *p = rowp + 4 * swz<CPR>(col >> 2, r) + (col & 3);
        if constexpr (C == 4) {
            const f4 v = *reinterpret_cast<const f4 *>(p);
            x[4 * c] = v.x; x[4 * c + 1] = v.y; x[4 * c + 2] = v.z; x[4 * c + 3] = v.w;
        } else {
            const f2 v = *reinterpret_cast<const f2 *>(p);
            x[2 * c] = v.x; x[2 * c + 1] = v.y;
        }
    }
}
