/* Measurement helpers of libkea_hip.so: kernels that measure what the MI355X sustains, so that benchmark figures can be
 * stated against measured peaks as well as against the published ones. They have no counterpart in the reference
 * (which quotes no measured peaks); their callers are the benchmark and the tests. Same conventions as
 * kea_lowbit.h: device pointers, a hipStream_t as void*, 0 on success, negative on a contract violation (nothing
 * launched, message in kea_last_error()), positive hipError_t on a launch failure. */
#ifndef KEA_PROBE_H
#define KEA_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Dense int8 matrix-core loop: `blocks` workgroups of four wave64s, each wave issuing `iters` rounds of eight
 * independent v_mfma_i32_16x16x64_i8 (32768 int8 ops each) on register operands, then one int32 per thread to
 * `out` (blocks * 256 ints: the wrapping sum of the thread's accumulator elements, so the work is not dead code and
 * its result can be checked). Ops per launch: blocks * 4 * iters * 8 * 32768.
 * blocks in [1, 65536], iters in [1, 1 << 20]. */
int kea_probe_mfma_i8(int64_t blocks, int64_t iters, int32_t *out, void *stream);

/* The ops one kea_probe_mfma_i8 launch performs (0 for arguments it would reject). */
int64_t kea_probe_mfma_i8_ops(int64_t blocks, int64_t iters);

#ifdef __cplusplus
}
#endif

#endif /* KEA_PROBE_H */
