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
//     dV^T) use the "row-owner" layout: output row i (0..15) of column tile it
//     (0..NT-1, NT = DP/16) is d = i * NT + it.  The A operand a lane needs for
//     one k-step -- row i = l16 of every tile -- is then NT consecutive floats
//     of one row-major LDS row (128- or 64-bit reads, lds_run), and accumulator
//     row 4*grp + r holds NT consecutive d of one output row (store_run).
//   * Scores are kept transposed (keys on the M axis, queries on the N axis):
//     the C layout of S^T (lane = query column, 4 key rows per register group)
//     is then exactly the B-operand layout the P.V product needs, with key
//     4*grp + kk on k-step kk.  P never leaves registers.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));

#define DEVI __device__ __forceinline__

constexpr float kLog2e = 1.4426950408889634f;

DEVI f4 mfma16(float a, float b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

DEVI int lane_id() { return threadIdx.x & 63; }

DEVI float wave_xor(float v, int mask) { return __shfl_xor(v, mask, 64); }

DEVI float max4grp(float v) {  // max over the four lane groups sharing l16
    v = fmaxf(v, wave_xor(v, 16));
    v = fmaxf(v, wave_xor(v, 32));
    return v;
}
DEVI float sum4grp(float v) {
    v += wave_xor(v, 16);
    v += wave_xor(v, 32);
    return v;
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

// Reads the NT floats p[0..NT) (the row-owner A operand): 128-bit reads when
// NT % 4 == 0 (p then 16-byte aligned), else 64-bit reads.
template <int NT>
DEVI void lds_run(float (&x)[NT], const float *p) {
    if constexpr (NT % 4 == 0) {
#pragma unroll
        for (int i = 0; i < NT; i += 4) {
            const f4 v = *reinterpret_cast<const f4 *>(p + i);
            x[i] = v.x; x[i + 1] = v.y; x[i + 2] = v.z; x[i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < NT; i += 2) {
            const f2 v = *reinterpret_cast<const f2 *>(p + i);
            x[i] = v.x; x[i + 1] = v.y;
        }
    }
}

// Stores row r of row-owner accumulators, acc[it][r] * mul for it = 0..NT-1,
// to row[c0 .. c0 + NT), c0 = (4 grp + r) * NT; columns >= dim are dropped.
// 128-bit stores when rows are 16-byte aligned (vec4) and NT % 4 == 0, else
// 64-bit stores (dim and c0 are even, so a pair never straddles dim).
template <int NT>
DEVI void store_run(float *row, int c0, int dim, bool vec4, const f4 (&acc)[NT], int r, float mul) {
    if (NT % 4 == 0 && vec4) {
#pragma unroll
        for (int i = 0; i < NT; i += 4)
            if (c0 + i < dim)
                *reinterpret_cast<f4 *>(row + c0 + i) =
                    f4{acc[i][r], acc[i + 1][r], acc[i + 2][r], acc[i + 3][r]} * mul;
    } else {
#pragma unroll
        for (int i = 0; i < NT; i += 2)
            if (c0 + i < dim) *reinterpret_cast<f2 *>(row + c0 + i) = f2{acc[i][r], acc[i + 1][r]} * mul;
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

// Same from a swizzled unpadded tile (see swz): columns [c0, c0 + NT) of row r.
template <int NT, int CPR>
DEVI void lds_run_swz(float (&x)[NT], const float *tile, int r, int c0) {
    const float *rowp = tile + r * CPR * 4;
    if constexpr (NT % 4 == 0) {
#pragma unroll
        for (int i = 0; i < NT; i += 4) {
            const f4 v = *reinterpret_cast<const f4 *>(rowp + 4 * swz<CPR>((c0 + i) >> 2, r));
            x[i] = v.x; x[i + 1] = v.y; x[i + 2] = v.z; x[i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < NT; i += 2) {
            const int c = c0 + i;  // even: a 64-bit read never leaves its 16-byte chunk
            const f2 v = *reinterpret_cast<const f2 *>(rowp + 4 * swz<CPR>(c >> 2, r) + (c & 3));
            x[i] = v.x; x[i + 1] = v.y;
        }
    }
}

// Cooperative copy of `rows` rows x DP columns into LDS TRANSPOSED: element
// (r, c) lands at lds[c * LT + r] (LT = rows + 4).  Consecutive lanes take
// consecutive rows of one column chunk, so each scattered store of a wave hits
// consecutive banks; a later 128-bit read of lds[n * LT + 4g .. 4g+3] then
// yields four consecutive rows of column n, the A operand of four successive
// k-steps.  Rows >= nvalid and columns >= dim are written as zero.
template <int DP, int LT, int NT>
DEVI void stage_rows_t(float *lds, const float *g, size_t ld, int rows, int nvalid, int dim, bool vec4,
                       int tid) {
    if (vec4) {
        for (int e = tid; e < rows * (DP / 4); e += NT) {
            const int r = e % rows, c = (e / rows) * 4;
            f4 x = zero4();
            if (r < nvalid && c < dim) x = *reinterpret_cast<const f4 *>(g + (size_t)r * ld + c);
            lds[(c + 0) * LT + r] = x.x;
            lds[(c + 1) * LT + r] = x.y;
            lds[(c + 2) * LT + r] = x.z;
            lds[(c + 3) * LT + r] = x.w;
        }
    } else {
        for (int e = tid; e < rows * (DP / 2); e += NT) {
            const int r = e % rows, c = (e / rows) * 2;
            f2 x = f2{0.f, 0.f};
            if (r < nvalid && c < dim) x = *reinterpret_cast<const f2 *>(g + (size_t)r * ld + c);
            lds[(c + 0) * LT + r] = x.x;
            lds[(c + 1) * LT + r] = x.y;
        }
    }
}

// One global read, two LDS layouts: element (r, c) of a rows x DP block goes to
// rm[r * LW + c] (row-major, LW = DP + 4) and to tr[c * LT + r] (transposed,
// LT = rows + 4).  Consecutive lanes take consecutive rows of one column chunk:
// the row-major 128-bit stores then walk 4-bank steps (LW = DP + 4) and the
// transposed scalar stores consecutive banks.  Zero beyond nvalid rows / dim.
template <int DP, int LW, int LT, int NT>
DEVI void stage_rows_both(float *rm, float *tr, const float *g, size_t ld, int rows, int nvalid, int dim,
                          bool vec4, int tid) {
    if (vec4) {
        for (int e = tid; e < rows * (DP / 4); e += NT) {
            const int r = e % rows, c = (e / rows) * 4;
            f4 x = zero4();
            if (r < nvalid && c < dim) x = *reinterpret_cast<const f4 *>(g + (size_t)r * ld + c);
            *reinterpret_cast<f4 *>(rm + r * LW + c) = x;
            tr[(c + 0) * LT + r] = x.x;
            tr[(c + 1) * LT + r] = x.y;
            tr[(c + 2) * LT + r] = x.z;
            tr[(c + 3) * LT + r] = x.w;
        }
    } else {
        for (int e = tid; e < rows * (DP / 2); e += NT) {
            const int r = e % rows, c = (e / rows) * 2;
            f2 x = f2{0.f, 0.f};
            if (r < nvalid && c < dim) x = *reinterpret_cast<const f2 *>(g + (size_t)r * ld + c);
            *reinterpret_cast<f2 *>(rm + r * LW + c) = x;
            tr[(c + 0) * LT + r] = x.x;
            tr[(c + 1) * LT + r] = x.y;
        }
    }
}
