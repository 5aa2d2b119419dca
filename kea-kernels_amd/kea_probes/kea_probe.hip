// Measurement helpers of the benchmark library libkea_probe.so (include/kea_probe.h), built beside the product library
// libkea_hip.so but not part of it: a dense int8 matrix-core loop that measures the sustained MFMA rate, the launch
// floors of a GEMM-shaped grid (an empty kernel, and kernels that only move a GEMM tile's bytes), the cost of a
// cross-workgroup exchange and a bounded spin that keeps host submission out of a timed region.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "../../include/kea_lowbit.h"  // status codes (KEA_E*)
#include "../../include/kea_probe.h"

namespace {

// The calling thread's last failure message (kea_probe_last_error), kept apart from the product library's.
thread_local std::string g_probe_error;

int fail(int code, const std::string &message) {
    g_probe_error = message;
    return code;
}

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kProbeChains = 8;            // independent accumulators per wave: covers the MFMA dependency latency
constexpr int64_t kOpsPerMfma = 16 * 16 * 64 * 2;

// Each lane's operands are distinct words: a fixed pattern of non-zero words, or (operands != nullptr) the caller's
// [128][4] int32 words (a for lanes 0-63, then b), e.g. random bytes like a GEMM's data: the matrix cores draw more
// power on such operands and the clock drops. The accumulators feed one int32 per thread. Integer MFMA wraps (no
// saturation), so any iteration count is well defined.
__global__ void __launch_bounds__(256) mfma_i8_loop(int iters, const v4i *operands, int32_t *out) {
    const int lane = threadIdx.x & 63;
    v4i a = {0x01020304 + lane, 0x05060708 - lane, 0x090A0B0C ^ lane, 0x0D0E0F10 + 3 * lane};
    v4i b = {0x11121314 - lane, 0x15161718 + lane, 0x191A1B1C ^ (lane << 8), 0x1D1E1F20 + 5 * lane};
    if (operands) {
        a = operands[lane];
        b = operands[64 + lane];
    }
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

// The same loop on v_mfma_i32_32x32x32_i8 (65536 int8 ops each, 16 accumulator registers per chain): the operands are
// the same 16 bytes per lane, which this instruction reads as 32 rows x 32 k instead of 16 rows x 64 k.
typedef int v16i __attribute__((ext_vector_type(16)));
__global__ void __launch_bounds__(256) mfma_i8_loop32(int iters, const v4i *operands, int32_t *out) {
    const int lane = threadIdx.x & 63;
    v4i a = {0x01020304 + lane, 0x05060708 - lane, 0x090A0B0C ^ lane, 0x0D0E0F10 + 3 * lane};
    v4i b = {0x11121314 - lane, 0x15161718 + lane, 0x191A1B1C ^ (lane << 8), 0x1D1E1F20 + 5 * lane};
    if (operands) {
        a = operands[lane];
        b = operands[64 + lane];
    }
    v16i acc[kProbeChains];
#pragma unroll
    for (int c = 0; c < kProbeChains; ++c) {
        acc[c] = (v16i){};
        acc[c][0] = c;
    }
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int c = 0; c < kProbeChains; ++c) acc[c] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, acc[c], 0, 0, 0);
    }
    uint32_t s = 0;  // wrapping sum
#pragma unroll
    for (int c = 0; c < kProbeChains; ++c)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += (uint32_t)acc[c][r];
    out[(int64_t)blockIdx.x * 256 + threadIdx.x] = (int32_t)s;
}

bool probe_args_ok(int64_t blocks, int64_t iters) {
    return blocks >= 1 && blocks <= 65536 && iters >= 1 && iters <= (1 << 20);
}

// ---- launch floors ------------------------------------------------------------------------------------------------
// One workgroup of 256 threads per BM x BN output tile of an M x N x K GEMM, as the GEMM launches them. The data
// kinds move exactly one GEMM tile's operand bytes: the BM activation rows (BM * K bytes) and the BN weight columns'
// native 1-bit words (BN * K / 8 bytes, one contiguous range per tile) by direct global -> LDS copies, all issued
// before the first wait; and/or the tile's fp16 outputs (BM * BN * 2 bytes) by 8-byte stores.
struct FloorArgs {
    const int8_t *a;
    const uint8_t *w;
    uint16_t *y;
    long long ldy;
    int k, bm, bn;
    int a_units, w_units;  // 16-byte units per tile
};

typedef __attribute__((address_space(1))) const void *gptr_t;
typedef __attribute__((address_space(3))) void *lptr_t;

template <int KIND>
__global__ void __launch_bounds__(1024) floor_kernel(FloorArgs f) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    if constexpr (KIND == KEA_PROBE_EMPTY) {
        return;
    } else {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const int n0 = blockIdx.x * f.bn, m0 = blockIdx.y * f.bm;
        if constexpr (KIND & KEA_PROBE_LOADS) {
            const int row_units = f.k / 16;
            const int8_t *abase = f.a + (long long)m0 * f.k;
            const uint8_t *wbase = f.w + (long long)n0 * (f.k / 8);
            // unit u of the tile: activation units first, then weight units; a wave's 64 lanes fill 1 KiB of LDS
            for (int base = wave * 64; base < f.a_units + f.w_units; base += (int)blockDim.x) {
                const int u = base + lane;
                if (u < f.a_units) {
                    const int r = u / row_units, c = u - r * row_units;
                    __builtin_amdgcn_global_load_lds((gptr_t)(abase + (long long)r * f.k + c * 16),
                                                     (lptr_t)(lds + base * 16), 16, 0, 0);
                } else if (u < f.a_units + f.w_units) {
                    __builtin_amdgcn_global_load_lds((gptr_t)(wbase + (long long)(u - f.a_units) * 16),
                                                     (lptr_t)(lds + base * 16), 16, 0, 0);
                }
            }
            __builtin_amdgcn_s_waitcnt(0);  // every copy landed (vmcnt, expcnt, lgkmcnt all 0)
            __syncthreads();
        }
        if constexpr (KIND & KEA_PROBE_STORES) {
            const int groups = f.bn / 4, total = f.bm * groups;
            const int lds_words = (f.a_units + f.w_units) * 2;  // 8-byte words in LDS (data kinds with loads)
            for (int g = threadIdx.x; g < total; g += (int)blockDim.x) {
                const int r = g / groups, c = (g - r * groups) * 4;
                uint2 v = make_uint2(0u, 0u);
                if constexpr (KIND & KEA_PROBE_LOADS) v = ((const uint2 *)lds)[g % lds_words];
                *(uint2 *)(f.y + (long long)(m0 + r) * f.ldy + n0 + c) = v;
            }
        }
    }
}

// ---- cross-workgroup exchange -------------------------------------------------------------------------------------
// What it costs one launch to hand data from workgroups to the last-arriving workgroup of their group, the pattern an
// in-launch split-K reduction or a quantizer fused after a GEMM would need. Workgroup w writes `words` uint4 to its
// slot (word i = {w, i, w ^ i, 1}); then, by KIND, thread 0 counts the workgroup in on its group's counter. No
// workgroup waits for another, so every launch ends.
template <int KIND>
__global__ void __launch_bounds__(256) exchange_kernel(uint4 *slots, int words, int group, uint32_t *counters,
                                                       uint32_t *result) {
    const int w = blockIdx.x, nwg = gridDim.x;
    uint4 *mine = slots + (size_t)w * words;
    for (int i = threadIdx.x; i < words; i += 256) mine[i] = make_uint4((unsigned)w, (unsigned)i, (unsigned)(w ^ i), 1u);
    if constexpr (KIND == KEA_EXCHANGE_WRITE) {
        return;
    } else {
        const int g = w / group, first = g * group, members = min(group, nwg - first);
        __shared__ int last;
        __syncthreads();  // every thread's slot words are written (and, at workgroup scope, ordered) before the count
        if (threadIdx.x == 0) {
            unsigned old;
            if constexpr (KIND == KEA_EXCHANGE_FENCED)
                old = __hip_atomic_fetch_add(counters + g, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
            else
                old = __hip_atomic_fetch_add(counters + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            last = old == (unsigned)members - 1;
            if (last) __hip_atomic_store(counters + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if constexpr (KIND == KEA_EXCHANGE_FENCED) {
            if (!last) return;
            unsigned sum = 0;
            for (int v = threadIdx.x; v < members; v += 256) sum += slots[(size_t)(first + v) * words + words - 1].x;
            if (sum) atomicAdd(result, sum);
        }
    }
}

// Spins one wavefront on the constant-rate wall clock (s_memrealtime) until `ticks` have passed: always ends.
__global__ void __launch_bounds__(64) spin_kernel(unsigned long long ticks) {
    const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
    while (__builtin_amdgcn_s_memrealtime() - t0 < ticks) __builtin_amdgcn_s_sleep(4);
}

}  // namespace

extern "C" {

const char *kea_probe_last_error(void) { return g_probe_error.c_str(); }

int64_t kea_probe_mfma_i8_ops(int64_t blocks, int64_t iters) {
    if (!probe_args_ok(blocks, iters)) return 0;
    return blocks * 4 * iters * kProbeChains * kOpsPerMfma;
}

int kea_probe_mfma_i8_operands(int64_t blocks, int64_t iters, const int32_t *operands, int32_t *out, void *stream) {
    if (!probe_args_ok(blocks, iters))
        return fail(KEA_EINVAL, "kea_probe_mfma_i8: blocks must be in [1, 65536] and iters in [1, 2^20]");
    if (!out) return fail(KEA_EINVAL, "kea_probe_mfma_i8: out is null");
    if ((uintptr_t)out & 3) return fail(KEA_EALIGN, "kea_probe_mfma_i8: out must be 4-byte aligned");
    if ((uintptr_t)operands & 15) return fail(KEA_EALIGN, "kea_probe_mfma_i8: operands must be 16-byte aligned");
    hipLaunchKernelGGL(mfma_i8_loop, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, (int)iters,
                       (const v4i *)operands, out);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail((int)e, std::string("kea_probe_mfma_i8: ") + hipGetErrorString(e));
    return 0;
}

int kea_probe_mfma_i8(int64_t blocks, int64_t iters, int32_t *out, void *stream) {
    return kea_probe_mfma_i8_operands(blocks, iters, nullptr, out, stream);
}

int64_t kea_probe_mfma_i8_32_ops(int64_t blocks, int64_t iters) { return 2 * kea_probe_mfma_i8_ops(blocks, iters); }

int kea_probe_mfma_i8_32(int64_t blocks, int64_t iters, const int32_t *operands, int32_t *out, void *stream) {
    if (!probe_args_ok(blocks, iters))
        return fail(KEA_EINVAL, "kea_probe_mfma_i8_32: blocks must be in [1, 65536] and iters in [1, 2^20]");
    if (!out) return fail(KEA_EINVAL, "kea_probe_mfma_i8_32: out is null");
    if ((uintptr_t)out & 3) return fail(KEA_EALIGN, "kea_probe_mfma_i8_32: out must be 4-byte aligned");
    if ((uintptr_t)operands & 15) return fail(KEA_EALIGN, "kea_probe_mfma_i8_32: operands must be 16-byte aligned");
    hipLaunchKernelGGL(mfma_i8_loop32, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, (int)iters,
                       (const v4i *)operands, out);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail((int)e, std::string("kea_probe_mfma_i8_32: ") + hipGetErrorString(e));
    return 0;
}

int kea_probe_spin(int64_t ns, void *stream) {
    if (ns < 0 || ns > 100000000LL) return fail(KEA_EINVAL, "kea_probe_spin: ns must be in [0, 1e8]");
    int dev = 0, khz = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e == hipSuccess) e = hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev);
    if (e != hipSuccess) return fail((int)e, std::string("kea_probe_spin: ") + hipGetErrorString(e));
    if (khz <= 0) return fail(KEA_ENODEV, "kea_probe_spin: the device reports no wall-clock rate");
    const unsigned long long ticks = (unsigned long long)(ns * (long long)khz / 1000000LL);
    hipLaunchKernelGGL(spin_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, ticks);
    e = hipGetLastError();
    if (e != hipSuccess) return fail((int)e, std::string("kea_probe_spin: ") + hipGetErrorString(e));
    return 0;
}

int kea_probe_exchange(int kind, int64_t workgroups, int64_t words, int64_t group, void *slots, uint32_t *counters,
                       uint32_t *result, void *stream) {
    if (kind < KEA_EXCHANGE_WRITE || kind > KEA_EXCHANGE_FENCED)
        return fail(KEA_EINVAL, "kea_probe_exchange: kind must be 0 (write), 1 (count) or 2 (fenced)");
    if (workgroups < 1 || workgroups > 65536 || words < 1 || words > 65536 || group < 1 || group > workgroups)
        return fail(KEA_EINVAL, "kea_probe_exchange: workgroups and words must be in [1, 65536], group in "
                                     "[1, workgroups]");
    if (!slots || ((uintptr_t)slots & 15)) return fail(KEA_EALIGN, "kea_probe_exchange: slots must be 16-byte aligned");
    if (kind != KEA_EXCHANGE_WRITE && (!counters || ((uintptr_t)counters & 3)))
        return fail(KEA_EINVAL, "kea_probe_exchange: counting kinds need 4-byte aligned counters");
    if (kind == KEA_EXCHANGE_FENCED && (!result || ((uintptr_t)result & 3)))
        return fail(KEA_EINVAL, "kea_probe_exchange: the fenced kind needs a 4-byte aligned result");
    hipStream_t st = (hipStream_t)stream;
    void (*fn)(uint4 *, int, int, uint32_t *, uint32_t *) =
        kind == KEA_EXCHANGE_WRITE ? exchange_kernel<KEA_EXCHANGE_WRITE>
        : kind == KEA_EXCHANGE_COUNT ? exchange_kernel<KEA_EXCHANGE_COUNT>
                                     : exchange_kernel<KEA_EXCHANGE_FENCED>;
    hipLaunchKernelGGL(fn, dim3((unsigned)workgroups), dim3(256), 0, st, (uint4 *)slots, (int)words, (int)group,
                       counters, result);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail((int)e, std::string("kea_probe_exchange: ") + hipGetErrorString(e));
    return 0;
}

int kea_probe_floor(int kind, int64_t m, int64_t n, int64_t k, int bm, int bn, const int8_t *a, const uint32_t *w,
                    uint16_t *y, int64_t ldy, void *stream) {
    return kea_probe_floor_waves(kind, m, n, k, bm, bn, 4, a, w, y, ldy, stream);
}

int kea_probe_floor_waves(int kind, int64_t m, int64_t n, int64_t k, int bm, int bn, int waves, const int8_t *a,
                          const uint32_t *w, uint16_t *y, int64_t ldy, void *stream) {
    if (waves < 1 || waves > 16) return fail(KEA_EINVAL, "kea_probe_floor: waves must be in [1, 16]");
    if (kind < KEA_PROBE_EMPTY || kind > (KEA_PROBE_LOADS | KEA_PROBE_STORES))
        return fail(KEA_EINVAL, "kea_probe_floor: kind must be 0 (empty), 1 (loads), 2 (stores) or 3 (both)");
    if (bm < 16 || bm > 256 || bm % 16 || bn < 16 || bn > 256 || bn % 16)
        return fail(KEA_EINVAL, "kea_probe_floor: bm and bn must be multiples of 16 in [16, 256]");
    if (m < bm || n < bn || k < 128 || m % bm || n % bn || k % 128 || m > (1 << 20) || n > (1 << 20) || k > (1 << 16))
        return fail(KEA_EINVAL, "kea_probe_floor: m, n must be multiples of bm, bn (<= 2^20) and k a multiple of "
                                     "128 (<= 65536)");
    const long long a_units = (long long)bm * k / 16, w_units = (long long)bn * k / 128;
    const long long lds = (kind & KEA_PROBE_LOADS) ? (a_units + w_units) * 16 : 0;
    if (lds > 160 * 1024) return fail(KEA_EINVAL, "kea_probe_floor: bm * k + bn * k / 8 exceeds 160 KiB of LDS");
    if ((kind & KEA_PROBE_LOADS) && (!a || !w || ((uintptr_t)a & 15) || ((uintptr_t)w & 15)))
        return fail(KEA_EINVAL, "kea_probe_floor: loads need 16-byte aligned a [m, k] and w (native words)");
    if ((kind & KEA_PROBE_STORES) && (!y || ((uintptr_t)y & 7) || ldy < n || ldy % 4))
        return fail(KEA_EINVAL, "kea_probe_floor: stores need an 8-byte aligned fp16 y [m, ldy >= n], ldy % 4 == 0");
    FloorArgs f = {a, (const uint8_t *)w, y, (long long)ldy, (int)k, bm, bn, (int)a_units, (int)w_units};
    const dim3 grid((unsigned)(n / bn), (unsigned)(m / bm));
    hipStream_t st = (hipStream_t)stream;
    void (*fn)(FloorArgs) = kind == KEA_PROBE_EMPTY ? floor_kernel<KEA_PROBE_EMPTY>
                          : kind == KEA_PROBE_LOADS ? floor_kernel<KEA_PROBE_LOADS>
                          : kind == KEA_PROBE_STORES ? floor_kernel<KEA_PROBE_STORES>
                                                     : floor_kernel<KEA_PROBE_LOADS | KEA_PROBE_STORES>;
    if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return fail((int)e, std::string("kea_probe_floor: ") + hipGetErrorString(e));
    }
    hipLaunchKernelGGL(fn, grid, dim3((unsigned)waves * 64), (size_t)lds, st, f);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail((int)e, std::string("kea_probe_floor: ") + hipGetErrorString(e));
    return 0;
}

}  // extern "C"
