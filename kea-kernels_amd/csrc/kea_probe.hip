// Measurement helpers (include/kea_probe.h): a dense int8 matrix-core loop that measures the sustained MFMA rate.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "../../include/kea_probe.h"
#include "kea_internal.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kProbeChains = 8;            // independent accumulators per wave: covers the MFMA dependency latency
constexpr int64_t kOpsPerMfma = 16 * 16 * 64 * 2;

// Each lane's operands are distinct, non-zero words so the products are not constant; the accumulators feed one
// int32 per thread. Integer MFMA wraps (no saturation), so any iteration count is well defined.
__global__ void __launch_bounds__(256) mfma_i8_loop(int iters, int32_t *out) {
    const int lane = threadIdx.x & 63;
    const v4i a = {0x01020304 + lane, 0x05060708 - lane, 0x090A0B0C ^ lane, 0x0D0E0F10 + 3 * lane};
    const v4i b = {0x11121314 - lane, 0x15161718 + lane, 0x191A1B1C ^ (lane << 8), 0x1D1E1F20 + 5 * lane};
    v4i acc[kProbeChains];
#pragma unroll
    for (int c = 0; c < kProbeChains; ++c) acc[c] = (v4i){c, 0, 0, 0};
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int c = 0; c < kProbeChains; ++c) acc[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, acc[c], 0, 0, 0);
    }
    uint32_t s = 0;  // wrapping sum
#pragma unroll
    for (int c = 0; c < kProbeChains; ++c)
#pragma unroll
        for (int r = 0; r < 4; ++r) s += (uint32_t)acc[c][r];
    out[(int64_t)blockIdx.x * 256 + threadIdx.x] = (int32_t)s;
}

bool probe_args_ok(int64_t blocks, int64_t iters) {
    return blocks >= 1 && blocks <= 65536 && iters >= 1 && iters <= (1 << 20);
}

}  // namespace

extern "C" {

int64_t kea_probe_mfma_i8_ops(int64_t blocks, int64_t iters) {
    if (!probe_args_ok(blocks, iters)) return 0;
    return blocks * 4 * iters * kProbeChains * kOpsPerMfma;
}

int kea_probe_mfma_i8(int64_t blocks, int64_t iters, int32_t *out, void *stream) {
    if (!probe_args_ok(blocks, iters))
        return kea::fail(KEA_EINVAL, "kea_probe_mfma_i8: blocks must be in [1, 65536] and iters in [1, 2^20]");
    if (!out) return kea::fail(KEA_EINVAL, "kea_probe_mfma_i8: out is null");
    if ((uintptr_t)out & 3) return kea::fail(KEA_EALIGN, "kea_probe_mfma_i8: out must be 4-byte aligned");
    hipLaunchKernelGGL(mfma_i8_loop, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, (int)iters, out);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return kea::fail((int)e, std::string("kea_probe_mfma_i8: ") + hipGetErrorString(e));
    return 0;
}

}  // extern "C"
