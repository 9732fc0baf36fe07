// Calibration probes for the roofline: what this device sustains, next to the
// datasheet peaks (FP32 MFMA 157.3 TFLOP/s, HBM 8 TB/s).
//
// zt_cal_mfma: two interleaved accumulation chains of v_mfma_f32_16x16x4_f32
// per wave (a single dependent chain leaves the pipe idle between
// back-to-back MFMAs); launched with four waves per SIMD it measures the
// sustained FP32 matrix rate.
// zt_cal_read: a grid-stride streaming read of a large buffer in 16-byte
// nontemporal loads, the access pattern of the decode kernel, reduced to one
// value per thread so the loads cannot be dropped.
// zt_cal_empty: does nothing; back-to-back launches of it measure what a
// launch alone costs on the device (the floor of a latency-bound kernel).
#include "common.h"
#include "args.h"

extern "C" __global__ void __launch_bounds__(256) zt_cal_mfma(CalArgs a) {
    f4 c0 = zero4(), c1 = zero4();
    const float x = 1.f + threadIdx.x * 1e-7f, y = 1e-3f;
    for (int it = 0; it < a.iters; ++it) {
        c0 = mfma16(x, y, c0);
        c1 = mfma16(x, y, c1);
    }
    const f4 s = c0 + c1;
    a.out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = s.x + s.y + s.z + s.w;
}

extern "C" __global__ void __launch_bounds__(256) zt_cal_read(CalArgs a) {
    const f4 *x = reinterpret_cast<const f4 *>(a.src);
    f4 acc = zero4();
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < a.n4; i += (size_t)gridDim.x * blockDim.x)
        acc += __builtin_nontemporal_load(x + i);
    a.out[(size_t)blockIdx.x * blockDim.x + threadIdx.x] = acc.x + acc.y + acc.z + acc.w;
}

extern "C" __global__ void __launch_bounds__(1024) zt_cal_empty(CalArgs a) { (void)a; }
