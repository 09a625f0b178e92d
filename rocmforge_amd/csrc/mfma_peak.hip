// mfma_peak.hip -- MFMA peak microbenchmark (measurement only).
//
// The prefill GEMMs are priced against MI355X's published dense fp16 MFMA
// peak; this kernel measures what the chip sustains for the same instruction
// (v_mfma_f32_32x32x16_f16) when nothing else runs: every wave issues
// independent MFMAs on operands taken from the caller's data, alternating
// between two operand sets so the multiplier inputs switch from one MFMA to
// the next as they do in a GEMM.  The sustained rate depends on the data
// (switching activity sets the power draw and with it the clock), so the
// caller passes the operand distribution it wants priced.
#include "qk_common.h"

namespace rf {

typedef _Float16 pk_f16x8 __attribute__((ext_vector_type(8)));
typedef float pk_f32x16 __attribute__((ext_vector_type(16)));

constexpr int kPeakChains = 8;      // independent accumulators per wave

__global__ __launch_bounds__(256) void rf_mfma_peak_kernel(const uint16_t* __restrict__ a, float* __restrict__ out,
                                                           int iters) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    // two operand pairs per lane, 8 halves each, from the 4096-element pool
    auto ld = [&](int j) {
        return *reinterpret_cast<const pk_f16x8*>(a + (size_t)((t * 4 + j) * 8 & 4095));
    };
    const pk_f16x8 x0 = ld(0), y0 = ld(1), x1 = ld(2), y1 = ld(3);
    pk_f32x16 acc[kPeakChains];
#pragma unroll
    for (int j = 0; j < kPeakChains; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[j][e] = 0.0f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < kPeakChains; ++j)
            acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16((j & 1) ? x1 : x0, (j & 1) ? y1 : y0, acc[j], 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < kPeakChains; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) s += acc[j][e];
    out[t] = s;
}

}  // namespace rf

extern "C" hipError_t rf_mfma_peak_launch(const uint16_t* a, float* out, int grid, int iters, hipStream_t stream) {
    if (a == nullptr || out == nullptr || grid <= 0 || iters <= 0) return hipErrorInvalidValue;
    if (reinterpret_cast<uintptr_t>(a) & 15u) return hipErrorInvalidValue;
    hipLaunchKernelGGL(rf::rf_mfma_peak_kernel, dim3((unsigned)grid), dim3(256), 0, stream, a, out, iters);
    return hipGetLastError();
}
