// Device clock sample: each one-wave workgroup of the launch records which
// XCD it runs on, its hardware wave id (which names its CU), its CU's shader
// clock counter (s_memtime, core clock cycles) and the constant 100 MHz
// realtime counter (s_memrealtime). The cycle counters of different CUs are
// not aligned, so two samples on one stream around a stretch of work are
// compared CU by CU: 100 MHz * d(memtime) / d(realtime) is that CU's mean
// core clock over the stretch. The values go out through ordinary vector
// stores.
#include "kernels.h"

namespace h3a {
namespace {

__global__ __launch_bounds__(64) void clock_sample_kernel(uint64_t* out) {
    uint32_t xcc, hw;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
    const uint64_t cycles = __builtin_amdgcn_s_memtime();
    const uint64_t ticks = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) {
        uint64_t* o = out + 4 * blockIdx.x;
        o[0] = xcc & 0xfu;
        o[1] = hw;
        o[2] = cycles;
        o[3] = ticks;
    }
}

}  // namespace

hipError_t launch_clock_sample(uint64_t* out, hipStream_t stream) {
    hipLaunchKernelGGL(clock_sample_kernel, dim3(H3A_CLOCK_RECORDS), dim3(64), 0, stream, out);
    return hipGetLastError();
}

}  // namespace h3a
