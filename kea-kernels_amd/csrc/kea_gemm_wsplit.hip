// Launcher of the wave-split low-bit GEMM (kernel instances: kea_gemm_wsplit_p1.hip .. _p3.hip).
#include <hip/hip_runtime.h>

#include "kea_gemm_wsplit.h"

namespace kea {

hipError_t wsplit_prepare(const Params &p, int wbits, int parts, int tile, int s, int splits, bool sliced,
                          WsplitLaunch *out) {
    const WsplitTile &t = kWsplitTiles[tile];
    // unmasked vector loads need whole k-step ranges in every workgroup and complete weight quads (or one word);
    // bit-plane units are whole per k-step
    const bool planes = wsplit_planes(wbits, parts, t.rm, t.nt);
    const int ksteps = (p.K + 63) / 64, words = wbits == 1 ? s / 2 : s;
    const bool ragged = (p.K % 64) != 0 || ksteps % (t.nw * s) != 0 || (!planes && words > 1 && p.J % 4 != 0);
    const WsplitFn fn = parts == 1 ? wsplit_pick_p1(wbits, tile, s, sliced, ragged)
                      : parts == 2 ? wsplit_pick_p2(wbits, tile, s, sliced, ragged)
                                   : wsplit_pick_p3(wbits, tile, s, sliced, ragged);
    if (!fn) return hipErrorInvalidDeviceFunction;
    const int lds = wsplit_lds_bytes(wbits, parts, t);
    if (lds > 65536) {
        const hipError_t e = hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        if (e != hipSuccess) return e;
    }
    out->fn = fn;
    out->grid = dim3((unsigned)((p.N + t.nt * 16 - 1) / (t.nt * 16)), (unsigned)((p.M + t.rm * 16 - 1) / (t.rm * 16)),
                     (unsigned)splits);
    out->block = dim3(t.nw * 64);
    out->lds = lds;
    out->meta = (p.qs_dtype == KEA_F16 ? 1 : 0) | (p.ws_dtype == KEA_F16 ? 2 : 0) |
                (p.bias && p.bias_dtype == KEA_F16 ? 4 : 0);
    out->w_off = planes ? b1_plane_offset(p.N, p.K) : 0;  // the bit-plane part of the 1-bit layout, or its words
    return hipSuccess;
}

hipError_t wsplit_group_prepare(const Params &p, int wbits, int parts, int tile, int gq, int s, WsplitLaunch *out) {
    const WsplitTile &t = kWsplitTiles[tile];
    const WsplitFn fn = parts == 1 ? wsplit_group_pick_p1(wbits, tile, gq, s)
                      : parts == 2 ? wsplit_group_pick_p2(wbits, tile, gq, s)
                                   : wsplit_group_pick_p3(wbits, tile, gq, s);
    if (!fn) return hipErrorInvalidDeviceFunction;
    const int lds = wsplit_group_lds_bytes(parts, t, s, gq);
    if (lds > 65536) {
        const hipError_t e = hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        if (e != hipSuccess) return e;
    }
    out->fn = fn;
    out->grid = dim3((unsigned)((p.N + t.nt * 16 - 1) / (t.nt * 16)), (unsigned)((p.M + 15) / 16), 1u);
    out->block = dim3(t.nw * 64);
    out->lds = lds;
    // bit 3: alpha's rows are 16-byte aligned and whole 16-byte units (vector loads of the register-held alpha)
    const int esz = p.ws_dtype == KEA_F16 ? 2 : 4;
    const bool avec = ((uintptr_t)p.ws % 16 == 0) && ((long long)p.groups * esz) % 16 == 0;
    out->meta = (p.qs_dtype == KEA_F16 ? 1 : 0) | (p.ws_dtype == KEA_F16 ? 2 : 0) |
                (p.bias && p.bias_dtype == KEA_F16 ? 4 : 0) | (avec ? 8 : 0);
    out->w_off = 0;  // the word layout
    return hipSuccess;
}

}  // namespace kea
