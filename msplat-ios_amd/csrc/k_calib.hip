// k_calib.hip -- LDS access-pattern calibration (diagnostic).
//
// Reads LDS with one fixed pattern per launch so that rocprofv3's LDS
// counters (SQ_LDS_BANK_CONFLICT, SQ_LDS_IDX_ACTIVE) can be read against
// the measured time of the same accesses: each thread issues 2000 loads of
// W floats (W = 1, 2, 4: 4-, 8- and 16-byte accesses), eight independent
// loads per iteration so that the kernel is bound by LDS throughput, not
// latency.  Pattern p places lane l's access at
//   p = 0: W l            (consecutive lanes, consecutive accesses)
//   p = 1: 2 W l          (every other access)
//   p = 2: 4 W l
//   p = 3: 32 W l
//   p = 4: 0              (every lane the same address: a broadcast)
// inside a 64 KB array, each of the eight loads 1024 floats further on
// (wrapped), every address aligned to its width.
#include "kernels.h"

namespace {

constexpr int kLdsFloats = 16384;

template <int W>
__global__ __launch_bounds__(256) void k_lds_calib(int pattern, int iters, float *__restrict__ out) {
    __shared__ __align__(16) float s[kLdsFloats];
    for (int i = threadIdx.x; i < kLdsFloats; i += 256) s[i] = (float)i;
    __syncthreads();
    const int l = threadIdx.x & 63;
    const int stride = pattern == 0 ? 1 : pattern == 1 ? 2 : pattern == 2 ? 4 : pattern == 3 ? 32 : 0;
    int a = W * stride * l;
    constexpr int kMask = (kLdsFloats - 1) & ~(W - 1);
    float acc = 0.f;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int b = (a + u * 1024) & kMask;
            if constexpr (W == 4) {
                const float4 v = *reinterpret_cast<const float4 *>(&s[b]);
                acc += v.x + v.w;
            } else if constexpr (W == 2) {
                const float2 v = *reinterpret_cast<const float2 *>(&s[b]);
                acc += v.x + v.y;
            } else {
                acc += s[b];
            }
        }
        // the base is opaque to the compiler, so every load is issued
        asm volatile("" : "+v"(a));
    }
    out[blockIdx.x * 256 + threadIdx.x] = acc;
}

}  // namespace

namespace mskern {

int lds_calib_out_floats() { return kLdsCalibBlocks * 256; }

void launch_lds_calib(hipStream_t s, int bytes_per_lane, int pattern, float *out) {
    const int iters = kLdsCalibReads / 8;
    if (bytes_per_lane == 16)
        hipLaunchKernelGGL(k_lds_calib<4>, dim3(kLdsCalibBlocks), dim3(256), 0, s, pattern, iters, out);
    else if (bytes_per_lane == 8)
        hipLaunchKernelGGL(k_lds_calib<2>, dim3(kLdsCalibBlocks), dim3(256), 0, s, pattern, iters, out);
    else
        hipLaunchKernelGGL(k_lds_calib<1>, dim3(kLdsCalibBlocks), dim3(256), 0, s, pattern, iters, out);
}

}  // namespace mskern
