/* Measurement helpers of libkea_probe.so, the benchmark's own library (kea-kernels_amd/kea_probes/, built with
 * libkea_hip.so but not linked into it): kernels that measure what the MI355X sustains, so that benchmark figures can
 * be stated against measured peaks and launch floors as well as against the published peaks. They have no counterpart
 * in the reference (which quotes no measured peaks); their callers are bench.py and the tests. Same conventions as
 * kea_lowbit.h: device pointers, a hipStream_t as void*, 0 on success, negative KEA_E* status on a contract violation
 * (nothing launched, message in kea_probe_last_error()), positive hipError_t on a launch failure. */
#ifndef KEA_PROBE_H
#define KEA_PROBE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Message of the calling thread's last probe failure ("" if none). */
const char *kea_probe_last_error(void);

/* Dense int8 matrix-core loop: `blocks` workgroups of four wave64s, each wave issuing `iters` rounds of eight
 * independent v_mfma_i32_16x16x64_i8 (32768 int8 ops each) on register operands, then one int32 per thread to
 * `out` (blocks * 256 ints: the wrapping sum of the thread's accumulator elements, so the work is not dead code and
 * its result can be checked). Ops per launch: blocks * 4 * iters * 8 * 32768.
 * blocks in [1, 65536], iters in [1, 1 << 20]. */
int kea_probe_mfma_i8(int64_t blocks, int64_t iters, int32_t *out, void *stream);

/* The same loop on caller-supplied operands: `operands` is [128][4] int32 in device memory, 16-byte aligned (the A
 * operand words of lanes 0-63, then the B operand words), or NULL for kea_probe_mfma_i8's fixed pattern. Random bytes
 * measure the rate on data like a GEMM's: the matrix cores draw more power on them and the clock drops. */
int kea_probe_mfma_i8_operands(int64_t blocks, int64_t iters, const int32_t *operands, int32_t *out, void *stream);

/* The ops one kea_probe_mfma_i8 launch performs (0 for arguments it would reject). */
int64_t kea_probe_mfma_i8_ops(int64_t blocks, int64_t iters);

/* The same loop on v_mfma_i32_32x32x32_i8 (65536 int8 ops each; the same 16 operand bytes per lane, read as 32 rows x
 * 32 k), eight independent 16-register accumulators per wave, `operands` as for kea_probe_mfma_i8_operands (or NULL).
 * Ops per launch: kea_probe_mfma_i8_32_ops(blocks, iters) = blocks * 4 * iters * 8 * 65536. */
int kea_probe_mfma_i8_32(int64_t blocks, int64_t iters, const int32_t *operands, int32_t *out, void *stream);
int64_t kea_probe_mfma_i8_32_ops(int64_t blocks, int64_t iters);

/* Keeps the stream busy for `ns` nanoseconds (one wavefront spinning on the device's constant-rate wall clock, so
 * it always ends): enqueued in front of a timed region, it lets the host finish submitting the region's work before
 * the region's start event executes, so host submission latency stays out of the measurement. ns in [0, 1e8]. */
int kea_probe_spin(int64_t ns, void *stream);

/* Cross-workgroup exchange: `workgroups` workgroups of 256 threads in groups of `group` consecutive ones (the last
 * group may be shorter). Workgroup w writes `words` 16-byte words to its slot (slots: workgroups * words * 16 bytes,
 * 16-byte aligned; word i = {w, i, w ^ i, 1}), then:
 *   KEA_EXCHANGE_WRITE   nothing more (the cost of the writes alone);
 *   KEA_EXCHANGE_COUNT   counts itself in on its group's counter with a relaxed device-scope atomic (no ordering:
 *                        what the serialised arrivals on one address cost);
 *   KEA_EXCHANGE_FENCED  counts itself in with an acquire-release device-scope atomic, and the group's last arriver
 *                        reads the first component of every group member's last word and adds their sum to *result.
 * This is the exchange an in-launch split-K reduction (group = the K slices of a tile) or a quantizer fused behind a
 * GEMM (group = the column tiles of a row block) would need. counters: ceil(workgroups / group) uint32, zero before
 * the first launch; the counting kinds leave them zero. After one FENCED launch *result has grown by the sum of
 * 0 .. workgroups-1 (mod 2^32). workgroups and words in [1, 65536], group in [1, workgroups]. */
#define KEA_EXCHANGE_WRITE 0
#define KEA_EXCHANGE_COUNT 1
#define KEA_EXCHANGE_FENCED 2
int kea_probe_exchange(int kind, int64_t workgroups, int64_t words, int64_t group, void *slots, uint32_t *counters,
                       uint32_t *result, void *stream);

/* Launch floors of a GEMM-shaped grid: (n / bn) x (m / bm) workgroups of four wave64s, one per bm x bn output tile of
 * an m x n x k low-bit GEMM, as kea_lowbit_gemm launches them. What each workgroup does:
 *   KEA_PROBE_EMPTY    nothing (the dispatch and completion cost of the grid);
 *   KEA_PROBE_LOADS    copies its tile's operand bytes into LDS - the bm activation rows of a (int8 [m][k], bm * k
 *                      bytes) and the native 1-bit words of its bn weight columns (w, bn * k / 8 bytes) - every copy
 *                      issued before the first wait, then waits for all of them;
 *   KEA_PROBE_STORES   writes its bm x bn fp16 tile of y ([m][ldy]) with 8-byte stores (zeros);
 *   KEA_PROBE_LOADS | KEA_PROBE_STORES  both, the stored values read back from the loaded bytes.
 * Requirements: bm, bn multiples of 16 in [16, 256]; m, n multiples of bm, bn (<= 2^20); k a multiple of 128
 * (<= 65536); bm * k + bn * k / 8 <= 160 KiB when loading; a, w 16-byte aligned; y 8-byte aligned, ldy >= n,
 * ldy % 4 == 0. */
#define KEA_PROBE_EMPTY 0
#define KEA_PROBE_LOADS 1
#define KEA_PROBE_STORES 2
int kea_probe_floor(int kind, int64_t m, int64_t n, int64_t k, int bm, int bn, const int8_t *a, const uint32_t *w,
                    uint16_t *y, int64_t ldy, void *stream);

/* kea_probe_floor with `waves` wave64s per workgroup (in [1, 16]; kea_probe_floor uses 4). A workgroup's copies into
 * LDS go faster when more of its waves issue them, so a GEMM tile's floor is measured at the tile's own wave count. */
int kea_probe_floor_waves(int kind, int64_t m, int64_t n, int64_t k, int bm, int bn, int waves, const int8_t *a,
                          const uint32_t *w, uint16_t *y, int64_t ldy, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* KEA_PROBE_H */
