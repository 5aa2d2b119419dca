// Fused FastConformer encoder kernels for MI355X (gfx950), FP32: relative-position self-attention and the
// convolution module's GLU + depthwise convolution (BatchNorm folded into the depthwise weights by the caller).
//
// They replace the reference's Triton kernels `_attention` / `_position_scores` + `relative_attention`
// (kk/ternary/fused_kernels.py:163-240) and `_glu_pad` + the depthwise Conv1d of the patched convolution module
// (kk/ternary/layer_fusions4.py:10-30, :62-72). Arithmetic is IEEE FP32 (fused multiply-adds in the dot products);
// unlike the reference's online-softmax tiles, a workgroup holds whole score rows (T <= 256), so the softmax is the
// exact two-pass form.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "kea_internal.h"
#include "kea_merge.h"
#include "kea_wave.h"
#include "../../include/kea_encoder.h"

namespace {

constexpr int kQB = 8;        // query rows per workgroup
constexpr int kMaxT = 256;    // longest sequence a workgroup holds

using kea::wave_max;
using kea::wave_sum;

// One workgroup (256 threads, 4 waves) = one (batch b, head h, block of kQB = 8 query rows); wave w owns query rows
// 2w and 2w + 1. For query i and key j:
//   s[i][j] = ((q_i + u) . k_j + (q_i + v) . p_{T-1-i+j}) * scale,  a = softmax_j(s),  out_i = sum_j a[i][j] v_j
// q/k/v rows of token t live at qkv + (b*T + t) * ld + {0, H*DK, 2*H*DK} + h*DK; relative-position row r (r = 0 is
// position T-1) at pos + r * ldp + h*DK; out row at out + (b*T + t) * ldo + h*DK.
// Keys are padded to 64 * NK (lane l of a wave takes keys l + 64 n): the score phase keeps a wave's 2 x NK scores per
// lane in registers and does the softmax with wave reductions; padded keys are zero rows, masked to -inf. LDS holds
// qu / qv [8][DK], the probabilities [8][64 NK] and one row buffer [kQB - 1 + 64 NK][DK + 4] that holds K, then the
// positional rows, then V.
template <int DK, int NK>
__global__ void __launch_bounds__(256)
relpos_attention_kernel(const float *qkv, long long ld, const float *pos, long long ldp, const float *bias_u,
                        const float *bias_v, float *out, long long ldo, int T, int H, float scale) {
    constexpr int DP = DK + 4;                   // padded row: 16-byte aligned, rows spread over the banks
    constexpr int KP = 64 * NK;                  // padded key count
    constexpr int ROWS = kQB - 1 + KP;           // row buffer size (positional rows need kQB - 1 more)
    static_assert(DK == 128, "one float4 of the head dimension per lane in the P.V product");
    extern __shared__ __attribute__((aligned(16))) float sm[];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int b = blockIdx.z, h = blockIdx.y, i0 = blockIdx.x * kQB;
    float *qu = sm, *qv = sm + kQB * DK, *S = sm + 2 * kQB * DK, *R = S + kQB * KP;
    const float *qbase = qkv + (long long)b * T * ld + (long long)h * DK;
    const float *kbase = qbase + (long long)H * DK, *vbase = qbase + 2LL * H * DK;

    // queries with both biases: 8 x 128 floats = one float4 per thread
    {
        const int i = tid >> 5, d = (tid & 31) * 4, t = i0 + i;
        float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
        if (t < T) q = *(const float4 *)(qbase + (long long)t * ld + d);
        const float4 u = *(const float4 *)(bias_u + h * DK + d), v = *(const float4 *)(bias_v + h * DK + d);
        *(float4 *)(qu + i * DK + d) = make_float4(q.x + u.x, q.y + u.y, q.z + u.z, q.w + u.w);
        *(float4 *)(qv + i * DK + d) = make_float4(q.x + v.x, q.y + v.y, q.z + v.z, q.w + v.w);
    }

    // Rows [first, first + valid) of a [*, stride] matrix into buffer rows [0, valid), zeros in [valid, count);
    // batches of 8 float4 loads per thread are issued before their stores.
    auto stage = [&](const float *src, long long stride, int first, int valid, int count) {
        const int chunks = count * (DK / 4);
        for (int c0 = tid; c0 < chunks; c0 += 8 * 256) {
            float4 v[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int c = c0 + u * 256, r = c / (DK / 4), d = (c % (DK / 4)) * 4;
                v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (c < chunks && r < valid) v[u] = *(const float4 *)(src + (long long)(first + r) * stride + d);
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int c = c0 + u * 256, r = c / (DK / 4), d = (c % (DK / 4)) * 4;
                if (c < chunks) *(float4 *)(R + r * DP + d) = v[u];
            }
        }
    };

    const int ia = 2 * wave, ib = ia + 1;        // this wave's two query rows (block-relative)
    float sa[NK], sb[NK];                        // scores of rows ia / ib against keys lane + 64 n
#pragma unroll
    for (int n = 0; n < NK; ++n) sa[n] = sb[n] = 0.f;

    stage(kbase, ld, 0, T, KP);
    __syncthreads();
    for (int d = 0; d < DK; d += 4) {
        const float4 xa = *(const float4 *)(qu + ia * DK + d), xb = *(const float4 *)(qu + ib * DK + d);
#pragma unroll
        for (int n = 0; n < NK; ++n) {
            const float4 r = *(const float4 *)(R + (lane + 64 * n) * DP + d);
            sa[n] = __builtin_fmaf(xa.x, r.x, sa[n]); sa[n] = __builtin_fmaf(xa.y, r.y, sa[n]);
            sa[n] = __builtin_fmaf(xa.z, r.z, sa[n]); sa[n] = __builtin_fmaf(xa.w, r.w, sa[n]);
            sb[n] = __builtin_fmaf(xb.x, r.x, sb[n]); sb[n] = __builtin_fmaf(xb.y, r.y, sb[n]);
            sb[n] = __builtin_fmaf(xb.z, r.z, sb[n]); sb[n] = __builtin_fmaf(xb.w, r.w, sb[n]);
        }
    }
    __syncthreads();  // K no longer needed

    // positional rows: query i (block-relative) and key j use buffer row (ilast - i) + j, r = T-1-(i0+i)+j
    const int ilast = min(i0 + kQB, T) - 1 - i0;   // last valid block-relative query
    const int rlo = T - 1 - (i0 + ilast);
    stage(pos + (long long)h * DK, ldp, rlo, 2 * T - 1 - rlo, ROWS);
    __syncthreads();
    {
        const int oa = max(ilast - ia, 0), ob = max(ilast - ib, 0);  // rows past T never reach the output
        float pa[NK], pb[NK];
#pragma unroll
        for (int n = 0; n < NK; ++n) pa[n] = pb[n] = 0.f;
        for (int d = 0; d < DK; d += 4) {
            const float4 xa = *(const float4 *)(qv + ia * DK + d), xb = *(const float4 *)(qv + ib * DK + d);
#pragma unroll
            for (int n = 0; n < NK; ++n) {
                const float4 ra = *(const float4 *)(R + (oa + lane + 64 * n) * DP + d);
                const float4 rb = *(const float4 *)(R + (ob + lane + 64 * n) * DP + d);
                pa[n] = __builtin_fmaf(xa.x, ra.x, pa[n]); pa[n] = __builtin_fmaf(xa.y, ra.y, pa[n]);
                pa[n] = __builtin_fmaf(xa.z, ra.z, pa[n]); pa[n] = __builtin_fmaf(xa.w, ra.w, pa[n]);
                pb[n] = __builtin_fmaf(xb.x, rb.x, pb[n]); pb[n] = __builtin_fmaf(xb.y, rb.y, pb[n]);
                pb[n] = __builtin_fmaf(xb.z, rb.z, pb[n]); pb[n] = __builtin_fmaf(xb.w, rb.w, pb[n]);
            }
        }
        // softmax of the two rows (keys past T masked), probabilities to LDS
        float ma = -INFINITY, mb = -INFINITY;
#pragma unroll
        for (int n = 0; n < NK; ++n) {
            const bool valid = lane + 64 * n < T;
            sa[n] = valid ? (sa[n] + pa[n]) * scale : -INFINITY;
            sb[n] = valid ? (sb[n] + pb[n]) * scale : -INFINITY;
            ma = fmaxf(ma, sa[n]);
            mb = fmaxf(mb, sb[n]);
        }
        ma = wave_max(ma);
        mb = wave_max(mb);
        float za = 0.f, zb = 0.f;
#pragma unroll
        for (int n = 0; n < NK; ++n) {
            sa[n] = expf(sa[n] - ma);
            sb[n] = expf(sb[n] - mb);
            za = za + sa[n];
            zb = zb + sb[n];
        }
        const float inva = 1.0f / wave_sum(za), invb = 1.0f / wave_sum(zb);
#pragma unroll
        for (int n = 0; n < NK; ++n) {
            S[ia * KP + lane + 64 * n] = sa[n] * inva;
            S[ib * KP + lane + 64 * n] = sb[n] * invb;
        }
    }
    __syncthreads();  // probabilities complete, positional rows no longer needed

    stage(vbase, ld, 0, T, KP);
    __syncthreads();
    {
        // lane: 4 columns d0 .. d0+3 and the keys of one parity; the two parities are added at the end
        const int d0 = (lane & 31) * 4, par = lane >> 5;
        float4 oa = make_float4(0.f, 0.f, 0.f, 0.f), ob = oa;
        for (int j = par; j < T; j += 2) {
            const float a = S[ia * KP + j], c = S[ib * KP + j];
            const float4 v = *(const float4 *)(R + j * DP + d0);
            oa.x = __builtin_fmaf(a, v.x, oa.x); oa.y = __builtin_fmaf(a, v.y, oa.y);
            oa.z = __builtin_fmaf(a, v.z, oa.z); oa.w = __builtin_fmaf(a, v.w, oa.w);
            ob.x = __builtin_fmaf(c, v.x, ob.x); ob.y = __builtin_fmaf(c, v.y, ob.y);
            ob.z = __builtin_fmaf(c, v.z, ob.z); ob.w = __builtin_fmaf(c, v.w, ob.w);
        }
        oa.x = oa.x + __shfl_xor(oa.x, 32, 64); oa.y = oa.y + __shfl_xor(oa.y, 32, 64);
        oa.z = oa.z + __shfl_xor(oa.z, 32, 64); oa.w = oa.w + __shfl_xor(oa.w, 32, 64);
        ob.x = ob.x + __shfl_xor(ob.x, 32, 64); ob.y = ob.y + __shfl_xor(ob.y, 32, 64);
        ob.z = ob.z + __shfl_xor(ob.z, 32, 64); ob.w = ob.w + __shfl_xor(ob.w, 32, 64);
        const int t = i0 + (par ? ib : ia);  // lanes 0-31 store row ia, lanes 32-63 row ib
        const float4 o = make_float4(par ? ob.x : oa.x, par ? ob.y : oa.y, par ? ob.z : oa.z, par ? ob.w : oa.w);
        if (t < T) *(float4 *)(out + ((long long)b * T + t) * ldo + (long long)h * DK + d0) = o;
    }
}

typedef float v4f __attribute__((ext_vector_type(4)));

// Max / sum of R independent values over the 64 lanes of a wave (independent chains the scheduler interleaves).
template <int R>
__device__ __forceinline__ void wave_max_n(float *v) {
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] = wave_max(v[r]);
}
template <int R>
__device__ __forceinline__ void wave_sum_n(float *v) {
#pragma unroll
    for (int r = 0; r < R; ++r) v[r] = wave_sum(v[r]);
}

// Matrix-core form of the same attention for T <= 128 (one workgroup = 16 query rows of one (b, h), NW waves), on
// v_mfma_f32_16x16x4_f32: lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16] per step and ends with
// D[4 (l / 16) + r][l % 16]. A dot product over the head dimension takes d = 16 (s / 4) + 4 g + s % 4 at step s
// (g = l / 16 the k lane group): a lane's operands are 8 float4 loads straight from global memory, and the 4 lanes
// of a row read 64 contiguous bytes per load; any order of the 128 terms is the same dot product up to FP32
// rounding.
//   content scores   D = (q + u) K^T                      16 x 16 key tiles
//   position scores  D = (q + v) P_band^T                  the band of 16 + KP - 1 relative rows this block needs,
//                                                          taken back as bd[i][j] = band[i][j + 15 - i]
//   softmax          per row from LDS (exact two-pass, keys past T masked); a wave reduces its 16 / NW rows together
//   output           D^T = V^T probs^T over keys k = (KP/4) g + s: wave w owns 128 / NW head columns. With 4 waves
//                    they are two 16-row tiles, tile c holding columns 32 w + 2 j + c, so one float2 load of a V row
//                    per step feeds both tiles and each lane stores 8 consecutive output columns; with 8 waves one
//                    tile of columns 16 w + j.
// Every wave's score tiles (content tiles w, w + NW, ..., then position tiles w, w + NW, ...) run as one list whose
// next operand loads are issued before the current tile's MFMAs; the V operands are loaded at the start and consumed
// last. 8 waves halve a workgroup's serial MFMA work for grids too small to fill the CUs (batch 1).
template <int NKT, int NW, int SPLIT>
__global__ void __launch_bounds__(NW * 64)
relpos_attention_mfma_kernel(const float *qkv, long long ld, const float *pos, long long ldp, const float *bias_u,
                             const float *bias_v, float *out, long long ldo, int T, int H, float scale,
                             kea::SplitWs ws) {
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    static_assert(SPLIT == 1 || (SPLIT == 2 && NKT % 2 == 0), "two key halves need an even number of key tiles");
    constexpr int NKS = NKT / SPLIT;  // key tiles of this workgroup
    constexpr int DK = 128, KP = 16 * NKS, NPT = NKS + 1, KS = KP / 4, RPW = 16 / NW, VC = 128 / NW / 16;
    constexpr int SP = KP + 4, BP = 16 * NPT + 4;  // padded LDS row strides (floats)
    constexpr int NC = (NKS + NW - 1) / NW, NPOS = (NPT + NW - 1) / NW, NTASK = NC + NPOS;  // tiles per wave (max)
    constexpr int QP = DK + 4, KPL = (KP + 63) / 64;  // keys per lane in the softmax
    __shared__ __attribute__((aligned(16))) float Sc[16 * SP];
    __shared__ __attribute__((aligned(16))) float Bd[16 * BP];
    __shared__ __attribute__((aligned(16))) float Qu[16 * QP];
    __shared__ __attribute__((aligned(16))) float Qv[16 * QP];
    __shared__ float row_m[16], row_l[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 15, g = lane >> 4;
    // blockIdx.x is the head: consecutive workgroups go to different XCDs, so the query tiles (and key halves) of one
    // head share an XCD and its L2 serves their K, V and position rows after the first fetch
    const int b = blockIdx.z, h = blockIdx.x, qt = blockIdx.y / SPLIT, half = blockIdx.y % SPLIT, i0 = qt * 16;
    const int j0 = half * KP;  // first key of this workgroup
    const float *qbase = qkv + (long long)b * T * ld + (long long)h * DK;
    const float *kbase = qbase + (long long)H * DK, *vbase = qbase + 2LL * H * DK;

    // This wave's score tiles: task i < nc is content tile wave + NW i, then position tile wave + NW (i - nc).
    // DEPTH operand buffers: every tile's loads up front with 8 waves (at most 3 tiles a wave), one ahead with 4.
    constexpr int DEPTH = NW == 8 ? NTASK : 2;
    const int nc = max(NKS - wave + NW - 1, 0) / NW, npos = max(NPT - wave + NW - 1, 0) / NW;
    const int rbase = T - 1 - (i0 + 15) + j0;  // relative row of this workgroup's band position 0
    float kb[DEPTH][32];
    auto load_task = [&](int i, float *dst) {
        const bool content = i < nc;
        const int tile = wave + NW * (content ? i : i - nc);
        const int row = content ? j0 + tile * 16 + li : rbase + tile * 16 + li;
        const bool valid = i < nc + npos && (content ? row < T : (row >= 0 && row <= 2 * T - 2));
        const float *src = content ? kbase + (long long)row * ld : pos + (long long)row * ldp + (long long)h * DK;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (valid) v = *(const float4 *)(src + 16 * c + 4 * g);
            dst[4 * c] = v.x; dst[4 * c + 1] = v.y; dst[4 * c + 2] = v.z; dst[4 * c + 3] = v.w;
        }
    };
#pragma unroll
    for (int i = 0; i < DEPTH; ++i)
        if (i < NTASK) load_task(i, kb[i]);

    // V operands of the output phase: V[j0 + KS g + s][(128 / NW) wave + VC li .. + VC - 1] (zero for keys >= T)
    float vr[KS][VC];
#pragma unroll
    for (int st = 0; st < KS; ++st) {
        const int j = j0 + KS * g + st;
        const float *src = vbase + (long long)j * ld + (128 / NW) * wave + VC * li;
        if constexpr (VC == 2) {
            float2 v = make_float2(0.f, 0.f);
            if (j < T) v = *(const float2 *)src;
            vr[st][0] = v.x;
            vr[st][VC - 1] = v.y;
        } else {
            vr[st][0] = j < T ? *src : 0.f;
        }
    }

    // The 16 query rows with both position biases are formed once per workgroup in LDS (qu, qv [16][DK + 4]; every
    // wave reads its operands there instead of loading the rows again). Their loads go out after the wave's tile and
    // V loads, so all of a wave's memory traffic is in flight at once.
    for (int idx = tid; idx < 16 * (DK / 4); idx += NW * 64) {
        const int r = idx / (DK / 4), d = (idx % (DK / 4)) * 4, t = i0 + r;
        float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
        if (t < T) q = *(const float4 *)(qbase + (long long)t * ld + d);
        const float4 u = *(const float4 *)(bias_u + h * DK + d), v = *(const float4 *)(bias_v + h * DK + d);
        *(float4 *)(Qu + r * QP + d) = make_float4(q.x + u.x, q.y + u.y, q.z + u.z, q.w + u.w);
        *(float4 *)(Qv + r * QP + d) = make_float4(q.x + v.x, q.y + v.y, q.z + v.z, q.w + v.w);
    }

    // query operands: row li of qu / qv, columns 16 c + 4 g .. + 3 for c = 0..7
    __syncthreads();
    float qa[32], qb[32];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const float4 a = *(const float4 *)(Qu + li * QP + 16 * c + 4 * g);
        const float4 v = *(const float4 *)(Qv + li * QP + 16 * c + 4 * g);
        qa[4 * c] = a.x; qa[4 * c + 1] = a.y; qa[4 * c + 2] = a.z; qa[4 * c + 3] = a.w;
        qb[4 * c] = v.x; qb[4 * c + 1] = v.y; qb[4 * c + 2] = v.z; qb[4 * c + 3] = v.w;
    }

#pragma unroll
    for (int i = 0; i < NTASK; ++i) {
        if (i < nc + npos) {
            const bool content = i < nc;
            const int tile = wave + NW * (content ? i : i - nc);
            v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < 32; ++st)
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(content ? qa[st] : qb[st], kb[i % DEPTH][st], acc, 0, 0, 0);
            float *dst = content ? Sc + tile * 16 + li : Bd + tile * 16 + li;
            const int stride = content ? SP : BP;
#pragma unroll
            for (int r = 0; r < 4; ++r) dst[(4 * g + r) * stride] = acc[r];
        }
        if (i + DEPTH < NTASK) load_task(i + DEPTH, kb[i % DEPTH]);  // this tile's buffer is free again
    }
    __syncthreads();

    // softmax over this workgroup's keys: wave w owns rows RPW w .. RPW w + RPW - 1 (reduced together); lane takes
    // keys lane, lane + 64. One workgroup per row normalises; a key half keeps exp(s - max) and the row statistics.
    {
        float sv[RPW][KPL], mx[RPW], sum[RPW];
#pragma unroll
        for (int rr = 0; rr < RPW; ++rr) {
            const int i = RPW * wave + rr;
            mx[rr] = -INFINITY;
#pragma unroll
            for (int n = 0; n < KPL; ++n) {
                const int j = lane + 64 * n;
                sv[rr][n] = -INFINITY;
                if (j < KP && j0 + j < T) sv[rr][n] = (Sc[i * SP + j] + Bd[i * BP + j + 15 - i]) * scale;
                mx[rr] = fmaxf(mx[rr], sv[rr][n]);
            }
        }
        wave_max_n<RPW>(mx);
#pragma unroll
        for (int rr = 0; rr < RPW; ++rr) {
            sum[rr] = 0.f;
#pragma unroll
            for (int n = 0; n < KPL; ++n) {
                sv[rr][n] = expf(sv[rr][n] - mx[rr]);
                sum[rr] = sum[rr] + sv[rr][n];
            }
        }
        wave_sum_n<RPW>(sum);
#pragma unroll
        for (int rr = 0; rr < RPW; ++rr) {
            const int i = RPW * wave + rr;
            const float inv = SPLIT == 1 ? 1.0f / sum[rr] : 1.0f;
#pragma unroll
            for (int n = 0; n < KPL; ++n) {
                const int j = lane + 64 * n;
                if (j < KP) Sc[i * SP + j] = SPLIT == 1 ? sv[rr][n] * inv : sv[rr][n];
            }
            if (SPLIT > 1 && lane == 0) {
                row_m[i] = mx[rr];
                row_l[i] = sum[rr];
            }
        }
    }
    __syncthreads();

    // output: D^T[j][q] for the wave's two column tiles; B operand = probs[q = li][KS g + s]
    float pa[KS];
#pragma unroll
    for (int c = 0; c < KS; c += 4) {
        const float4 v = *(const float4 *)(Sc + li * SP + KS * g + c);
        pa[c] = v.x; pa[c + 1] = v.y; pa[c + 2] = v.z; pa[c + 3] = v.w;
    }
    v4f acc[VC];
#pragma unroll
    for (int c = 0; c < VC; ++c) acc[c] = (v4f){0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < KS; ++st)
#pragma unroll
        for (int c = 0; c < VC; ++c) acc[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(vr[st][c], pa[st], acc[c], 0, 0, 0);
    // lane holds rows j = 4 g + r for query q = li: column (128 / NW) w + VC (4 g + r) + c
    const int t = i0 + li;
    const long long col = (long long)h * DK + (128 / NW) * wave + 4 * VC * g;
    float o[4 * VC];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int c = 0; c < VC; ++c) o[VC * r + c] = acc[c][r];
    if constexpr (SPLIT > 1) {
        // this half's unnormalised partial and its rows' statistics; the consumer merges the halves
        if (t < T) {
            const long long rows = (long long)gridDim.z * T, row = (long long)b * T + t, hd = (long long)H * DK;
            float *po = ws.o + ((long long)half * rows + row) * hd + col;
#pragma unroll
            for (int v = 0; v < VC; ++v)
                *(float4 *)(po + 4 * v) = make_float4(o[4 * v], o[4 * v + 1], o[4 * v + 2], o[4 * v + 3]);
            if (wave == 0 && g == 0)
                *(float2 *)(ws.ml + (((long long)half * rows + row) * H + h) * 2) = make_float2(row_m[li], row_l[li]);
        }
        return;
    }
    if (t < T) {
        float *dst = out + ((long long)b * T + t) * ldo + col;
#pragma unroll
        for (int v = 0; v < VC; ++v) *(float4 *)(dst + 4 * v) = make_float4(o[4 * v], o[4 * v + 1], o[4 * v + 2], o[4 * v + 3]);
    }
}

// y[b][t][c] = bias[c] + sum_j w[c][j] * glu(x)[b][t + j - KW/2][c],  glu(x)[.][c] = x[.][c] * sigmoid(x[.][C + c]),
// zero outside [0, T). One thread per output element, threads along c (coalesced).
__global__ void __launch_bounds__(256)
glu_dwconv_kernel(const float *x, long long ldx, const float *w, const float *bias, float *y, long long ldy, int T,
                  int C, int KW) {
    const int c = blockIdx.x * 256 + threadIdx.x, t = blockIdx.y, b = blockIdx.z;
    if (c >= C) return;
    const int half = KW / 2;
    float acc = bias ? bias[c] : 0.f;
    for (int j = 0; j < KW; ++j) {
        const int tt = t + j - half;
        if (tt < 0 || tt >= T) continue;
        const float *row = x + ((long long)b * T + tt) * ldx;
        const float a = row[c], g = row[C + c];
        acc = __builtin_fmaf(w[c * KW + j], a * (1.0f / (1.0f + expf(-g))), acc);
    }
    y[((long long)b * T + t) * ldy + c] = acc;
}

// ---- dw-striding subsampling (x8): the convolution stack in front of the encoder layers -----------------------
//
// NeMo's dw_striding subsampling on [B, 1, T, F] (time rows, mel columns): conv 3x3/2 (1 -> C) + ReLU, then twice
// [depthwise 3x3/2 + pointwise 1x1 (C -> C) + ReLU], then flatten (c, f) and a linear layer. The pointwise convolutions
// and the linear layer are plain matrix products (PyTorch / rocBLAS); the kernels below are the rest.

// Front: conv 3x3/2 (1 input channel, padding 1) + bias + ReLU, then depthwise 3x3/2 (padding 1) + bias, without
// materialising the first convolution's [B, C, T1, F1] output. A thread owns one output position (t2, f2) and loops
// over a group of CG channels: it holds the 7 x 7 input patch its 3 x 3 first-convolution values need and recomputes
// them per channel (each first-convolution value feeds up to 4 outputs: 2.25x its FMAs, against a 4x larger tensor
// round trip through HBM). Channel weights are wave-uniform (scalar loads). x: [B][F][T] (mel-major, as the
// preprocessor writes it), y: [B][C][T2][F2].
constexpr int kSubTT = 8;   // output rows (t2) per workgroup; 256 threads = 8 rows x 32 columns
template <int CG>
__global__ void __launch_bounds__(256)
subsample_front_kernel(const float *x, int T, int F, const float *w1, const float *b1, const float *w2,
                       const float *b2, float *y, int C, int T1, int F1, int T2, int F2) {
    constexpr int XR = 4 * kSubTT + 3, XC = 132, XN = (XR * XC + 255) / 256;
    __shared__ float xt[XR][XC];          // input rows 4 t2a - 3 .. , columns -1 .. 130 (zero padded)
    __shared__ float4 wl[CG][5];          // per channel: w1[0..8], b1, w2[0..8], b2 (20 floats)
    const int b = blockIdx.z, c0 = blockIdx.y * CG, t2a = blockIdx.x * kSubTT;
    const int r0 = 4 * t2a - 3;
    const float *xb = x + (long long)b * F * T;
    {   // tile loads, consecutive threads along time (x is mel-major, time contiguous), all issued before the stores
        float v[XN];
#pragma unroll
        for (int u = 0; u < XN; ++u) {
            const int idx = threadIdx.x + 256 * u, j = idx / XR, i = idx % XR, r = r0 + i, c = j - 1;
            v[u] = (idx < XR * XC && r >= 0 && r < T && c >= 0 && c < F) ? xb[(long long)c * T + r] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < XN; ++u) {
            const int idx = threadIdx.x + 256 * u;
            if (idx < XR * XC) xt[idx % XR][idx / XR] = v[u];
        }
    }
    for (int idx = threadIdx.x; idx < CG * 20; idx += 256) {
        const int cc = idx / 20, e = idx % 20, c = min(c0 + cc, C - 1);
        ((float *)wl)[idx] = e < 9 ? w1[c * 9 + e] : e == 9 ? b1[c] : e < 19 ? w2[c * 9 + e - 10] : b2[c];
    }
    __syncthreads();
    const int t2 = t2a + threadIdx.x / 32, f2 = threadIdx.x % 32;
    // this thread's 7 x 7 patch: input rows 4 t2 - 3 + i, columns 4 f2 - 3 + j (tile column 4 f2 - 2 + j); the
    // first-convolution value at (2 t2 - 1 + dy, 2 f2 - 1 + dx) reads patch rows 2 dy + ky and columns 2 dx + kx
    float xin[7][7];
#pragma unroll
    for (int i = 0; i < 7; ++i)
#pragma unroll
        for (int j = 0; j < 7; ++j) {
            const int col = 4 * f2 - 2 + j;
            xin[i][j] = col >= 0 && col < 132 ? xt[4 * (threadIdx.x / 32) + i][col] : 0.f;
        }
    bool valid1[3][3];   // first-convolution positions inside [0, T1) x [0, F1) (outside: the depthwise padding)
#pragma unroll
    for (int dy = 0; dy < 3; ++dy)
#pragma unroll
        for (int dx = 0; dx < 3; ++dx) {
            const int r1 = 2 * t2 - 1 + dy, c1 = 2 * f2 - 1 + dx;
            valid1[dy][dx] = r1 >= 0 && r1 < T1 && c1 >= 0 && c1 < F1;
        }
    const bool live = t2 < T2 && f2 < F2;
#pragma unroll 2
    for (int cc = 0; cc < CG; ++cc) {
        const int c = c0 + cc;
        if (c >= C) break;
        float wv[20];
#pragma unroll
        for (int q = 0; q < 5; ++q) {
            const float4 f4 = wl[cc][q];
            wv[4 * q] = f4.x; wv[4 * q + 1] = f4.y; wv[4 * q + 2] = f4.z; wv[4 * q + 3] = f4.w;
        }
        const float *wa = wv, *wb = wv + 10;
        const float ba = wv[9];
        float acc = wv[19];
#pragma unroll
        for (int dy = 0; dy < 3; ++dy)
#pragma unroll
            for (int dx = 0; dx < 3; ++dx) {
                float h = ba;
#pragma unroll
                for (int ky = 0; ky < 3; ++ky)
#pragma unroll
                    for (int kx = 0; kx < 3; ++kx) h = __builtin_fmaf(wa[ky * 3 + kx], xin[2 * dy + ky][2 * dx + kx], h);
                h = valid1[dy][dx] ? fmaxf(h, 0.f) : 0.f;
                acc = __builtin_fmaf(wb[dy * 3 + dx], h, acc);
            }
        if (live) y[(((long long)b * C + c) * T2 + t2) * F2 + f2] = acc;
    }
}

// Depthwise 3x3/2 (padding 1) + bias on relu(x + in_bias[c]) (the previous pointwise convolution's bias and ReLU,
// applied on load). x: [B][C][H][W], y: [B][C][H2][W2]; one thread per output element.
__global__ void __launch_bounds__(256)
dwconv_s2_kernel(const float *x, const float *in_bias, const float *w, const float *bias, float *y, int C, int H,
                 int W, int H2, int W2, long long total) {
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= total) return;
    const int o = (int)(idx % W2), r = (int)((idx / W2) % H2);
    const long long bc = idx / ((long long)W2 * H2);
    const int c = (int)(bc % C);
    const float *xc = x + bc * H * W;
    const float ib = in_bias ? in_bias[c] : 0.f;
    float acc = bias[c];
#pragma unroll
    for (int ky = 0; ky < 3; ++ky)
#pragma unroll
        for (int kx = 0; kx < 3; ++kx) {
            const int rr = 2 * r - 1 + ky, cc = 2 * o - 1 + kx;
            if (rr < 0 || rr >= H || cc < 0 || cc >= W) continue;
            acc = __builtin_fmaf(w[c * 9 + ky * 3 + kx], fmaxf(xc[rr * W + cc] + ib, 0.f), acc);
        }
    y[idx] = acc;
}

// y[b][t][c * W + f] = relu(x[b][c][t][f] + bias[c]): the last pointwise convolution's bias and ReLU with the
// flatten of (channel, frequency) per time step.
__global__ void __launch_bounds__(256)
bias_relu_flatten_kernel(const float *x, const float *bias, float *y, int C, int H, int W, long long total) {
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;  // over y
    if (idx >= total) return;
    const int f = (int)(idx % W), c = (int)((idx / W) % C), t = (int)((idx / ((long long)W * C)) % H);
    const long long b = idx / ((long long)W * C * H);
    y[idx] = fmaxf(x[((b * C + c) * H + t) * W + f] + bias[c], 0.f);
}

// STFT frames as torch.stft builds them for center = True, pad_mode "constant": frame f of clip b is the window times
// the pre-emphasised audio from f * hop - n_fft / 2, zero outside the clip. One thread per frame element; the
// pre-emphasis is the same two roundings (product, then difference) as a[i] - preemph * a[i-1] in FP32.
__global__ void __launch_bounds__(256)
stft_frames_kernel(const float *audio, long long samples, float preemph, const float *window, int n_fft, int hop,
                   long long frames, float *out) {
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long per_clip = frames * n_fft;
    const long long b = blockIdx.y;
    if (idx >= per_clip) return;
    const long long f = idx / n_fft;
    const int j = (int)(idx - f * n_fft);
    const long long i = f * hop + j - n_fft / 2;
    const float *a = audio + b * samples;
    float x = 0.f;
    if (i == 0) {
        x = a[0];
    } else if (i > 0 && i < samples) {
        const float prev = preemph * a[i - 1];
        x = a[i] - prev;
    }
    out[b * per_clip + idx] = window[j] * x;
}

// Log-mel features with per-feature normalisation over time, one workgroup per (clip, mel bin):
//   v[t] = log(sum_{k in [lo, hi)} fb[m][k] * (re^2 + im^2)[k][t] + log_eps)       (the filter's nonzero bins only)
//   y[t] = (v[t] - mean) / (std + std_eps),  mean over the frames, std with the n - 1 divisor
// spec: interleaved complex [B][bins][ld_t]; y: [B][mels][frames]. Thread th owns frames th, th + 256, ...: it
// writes v, re-reads its own elements for the variance and the normalisation (no barrier between those passes).
__global__ void __launch_bounds__(256)
logmel_normalize_kernel(const float2 *spec, int bins, int frames, long long ld_t, const float *fb, const int *lo,
                        const int *hi, int mels, float log_eps, float std_eps, float *y) {
    __shared__ float red[2][4];
    const int m = blockIdx.x, b = blockIdx.y, th = threadIdx.x, wave = th >> 6;
    const float2 *sb = spec + (long long)b * bins * ld_t;
    float *yr = y + ((long long)b * mels + m) * frames;
    const int k0 = lo[m], k1 = hi[m];
    float sum = 0.f;
    for (int t0 = 0; t0 < frames; t0 += 1024) {   // 4 frames per thread per chunk; 4 bins x 4 frames loads in flight
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        for (int k = k0; k < k1; k += 4) {
            float2 c[4][4];
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int t = t0 + th + 256 * i;
                    c[kk][i] = make_float2(0.f, 0.f);
                    if (k + kk < k1 && t < frames) c[kk][i] = sb[(long long)(k + kk) * ld_t + t];
                }
#pragma unroll
            for (int kk = 0; kk < 4; ++kk) {
                const float w = k + kk < k1 ? fb[m * bins + k + kk] : 0.f;
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    acc[i] = __builtin_fmaf(w, c[kk][i].x * c[kk][i].x + c[kk][i].y * c[kk][i].y, acc[i]);
            }
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = t0 + th + 256 * i;
            if (t < frames) {
                const float v = logf(acc[i] + log_eps);
                yr[t] = v;
                sum = sum + v;
            }
        }
    }
    sum = wave_sum(sum);
    if ((th & 63) == 0) red[0][wave] = sum;
    __syncthreads();
    const float mean = ((red[0][0] + red[0][1]) + (red[0][2] + red[0][3])) / (float)frames;
    float sq = 0.f;
    for (int t = th; t < frames; t += 256) {
        const float d = yr[t] - mean;
        sq = __builtin_fmaf(d, d, sq);
    }
    sq = wave_sum(sq);
    if ((th & 63) == 0) red[1][wave] = sq;
    __syncthreads();
    const float var = ((red[1][0] + red[1][1]) + (red[1][2] + red[1][3])) / (float)(frames > 1 ? frames - 1 : 1);
    const float inv = 1.0f / (sqrtf(var) + std_eps);
    for (int t = th; t < frames; t += 256) yr[t] = (yr[t] - mean) * inv;
}

// The same features from a frame-major spectrum ([B][ld_f][bins], the real FFT of kea_stft_frames' rows). A filter's
// band of a frame is a few contiguous bins, so the band of kChunk frames is staged through LDS as power values,
// read with consecutive bins on consecutive lanes; each thread then sums its frames' powers in the order of
// logmel_normalize_kernel (increasing k, one fma per bin) and the normalisation is the same code, so both layouts give
// the same bits. Bands wider than kBand bins are staged kBand bins at a time.
constexpr int kChunk = 512, kBand = 16;
__global__ void __launch_bounds__(256)
logmel_normalize_frames_kernel(const float2 *spec, int bins, int frames, long long ld_f, const float *fb,
                               const int *lo, const int *hi, int mels, float log_eps, float std_eps, float *y) {
    __shared__ float pw[kBand * (kChunk + 1)];  // [bin of the band][frame], rows padded against bank conflicts
    __shared__ float red[2][4];
    const int m = blockIdx.x, b = blockIdx.y, th = threadIdx.x, wave = th >> 6;
    const float2 *sb = spec + (long long)b * ld_f * bins;
    float *yr = y + ((long long)b * mels + m) * frames;
    const int k0 = lo[m], k1 = hi[m];
    float sum = 0.f;
    for (int t0 = 0; t0 < frames; t0 += kChunk) {
        const int nf = min(kChunk, frames - t0);
        float acc[kChunk / 256];
#pragma unroll
        for (int i = 0; i < kChunk / 256; ++i) acc[i] = 0.f;
        for (int kc = k0; kc < k1; kc += kBand) {
            const int w = min(kBand, k1 - kc);
            __syncthreads();  // the previous band's readers are done
            for (int e = th; e < nf * w; e += 256) {
                const int f = e / w, kk = e - f * w;
                const float2 c = sb[(long long)(t0 + f) * bins + kc + kk];
                pw[kk * (kChunk + 1) + f] = c.x * c.x + c.y * c.y;
            }
            __syncthreads();
            for (int kk = 0; kk < w; ++kk) {
                const float wt = fb[m * bins + kc + kk];
#pragma unroll
                for (int i = 0; i < kChunk / 256; ++i)
                    acc[i] = __builtin_fmaf(wt, pw[kk * (kChunk + 1) + th + 256 * i], acc[i]);
            }
        }
#pragma unroll
        for (int i = 0; i < kChunk / 256; ++i) {
            const int t = t0 + th + 256 * i;
            if (t < frames) {
                const float v = logf(acc[i] + log_eps);
                yr[t] = v;
                sum = sum + v;
            }
        }
    }
    sum = wave_sum(sum);
    if ((th & 63) == 0) red[0][wave] = sum;
    __syncthreads();
    const float mean = ((red[0][0] + red[0][1]) + (red[0][2] + red[0][3])) / (float)frames;
    float sq = 0.f;
    for (int t = th; t < frames; t += 256) {
        const float d = yr[t] - mean;
        sq = __builtin_fmaf(d, d, sq);
    }
    sq = wave_sum(sq);
    if ((th & 63) == 0) red[1][wave] = sq;
    __syncthreads();
    const float var = ((red[1][0] + red[1][1]) + (red[1][2] + red[1][3])) / (float)(frames > 1 ? frames - 1 : 1);
    const float inv = 1.0f / (sqrtf(var) + std_eps);
    for (int t = th; t < frames; t += 256) yr[t] = (yr[t] - mean) * inv;
}

using kea::attention_splits;

int64_t split_ws_bytes(int64_t batch, int64_t t, int heads) { return 4 * kea::split_ws_floats(batch * t, heads); }

// out[row][k] = the merged halves; one thread per four features.
__global__ void __launch_bounds__(256)
attention_merge_kernel(kea::SplitWs ws, long long rows, int heads, float *out, long long ldo) {
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x, per_row = (long long)heads * 32;
    if (idx >= rows * per_row) return;
    const long long row = idx / per_row;
    const int k = (int)(idx - row * per_row) * 4;
    float v[4];
    kea::merged4(ws, rows, heads, row, k, v);
    *(float4 *)(out + row * ldo + k) = make_float4(v[0], v[1], v[2], v[3]);
}

int attention(const float *qkv, int64_t ld, const float *pos, int64_t ldp, const float *bias_u, const float *bias_v,
              float *out, int64_t ldo, int64_t batch, int64_t t, int heads, int head_dim, float scale, void *ws,
              int64_t ws_bytes, void *stream) {
    if (batch < 0 || t < 1 || heads < 1 || head_dim != 128 || batch > 65535 || heads > 65535)
        return kea::fail(KEA_EINVAL, "bad sizes (head_dim must be 128)");
    if (t > kMaxT) return kea::fail(KEA_EINVAL, "sequence longer than 256 frames: use the unfused attention");
    if (batch == 0) return KEA_OK;
    const bool split = ws && attention_splits(batch, t, heads);
    if (!qkv || !pos || !bias_u || !bias_v || (!out && !split)) return kea::fail(KEA_EINVAL, "null pointer");
    if (ld < 3LL * heads * head_dim || ldp < (int64_t)heads * head_dim || (out && ldo < (int64_t)heads * head_dim))
        return kea::fail(KEA_EINVAL, "leading dimension too small");
    if (((uintptr_t)qkv | (uintptr_t)pos | (uintptr_t)out | (uintptr_t)bias_u | (uintptr_t)bias_v) & 15 ||
        (ld | ldp | ldo) & 3)
        return kea::fail(KEA_EALIGN, "qkv, pos, out and the biases need 16-byte aligned rows");
    if (t <= 128) {
        const int nkt = (int)((t + 15) / 16);
        kea::SplitWs sw{nullptr, nullptr};
        if (split) {
            if (ws_bytes < split_ws_bytes(batch, t, heads))
                return kea::fail(KEA_ESPACE, "attention workspace too small: need " +
                                                 std::to_string(split_ws_bytes(batch, t, heads)) + " bytes");
            if ((uintptr_t)ws & 15) return kea::fail(KEA_EALIGN, "attention workspace must be 16-byte aligned");
            sw = kea::split_ws(ws, batch * t, heads);
        }
        const dim3 grid((unsigned)heads, (unsigned)(nkt * (split ? 2 : 1)), (unsigned)batch);
        void (*fn)(const float *, long long, const float *, long long, const float *, const float *, float *,
                   long long, int, int, float, kea::SplitWs) = nullptr;
        // 8 waves per workgroup when the grid leaves CUs idle (fewer workgroups than the 256 CUs)
        const bool wide = (long long)grid.x * grid.y * grid.z < 256;
#define KEA_ATT(N) fn = wide ? relpos_attention_mfma_kernel<N, 8, 1> : relpos_attention_mfma_kernel<N, 4, 1>
#define KEA_ATT2(N) fn = relpos_attention_mfma_kernel<N, 8, 2>
        if (split) {
            switch (nkt) {
                case 2: KEA_ATT2(2); break;
                case 4: KEA_ATT2(4); break;
                case 6: KEA_ATT2(6); break;
                default: KEA_ATT2(8); break;
            }
        } else {
            switch (nkt) {
                case 1: KEA_ATT(1); break;
                case 2: KEA_ATT(2); break;
                case 3: KEA_ATT(3); break;
                case 4: KEA_ATT(4); break;
                case 5: KEA_ATT(5); break;
                case 6: KEA_ATT(6); break;
                case 7: KEA_ATT(7); break;
                default: KEA_ATT(8); break;
            }
        }
#undef KEA_ATT
#undef KEA_ATT2
        hipLaunchKernelGGL(fn, grid, dim3(wide || split ? 512 : 256), 0, (hipStream_t)stream, qkv, (long long)ld, pos,
                           (long long)ldp, bias_u, bias_v, out, (long long)ldo, (int)t, heads, scale, sw);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return kea::fail((int)e, std::string("attention launch failed: ") + hipGetErrorString(e));
        if (split && out) {
            const long long rows = batch * t, work = rows * heads * 32;
            hipLaunchKernelGGL(attention_merge_kernel, dim3((unsigned)((work + 255) / 256)), dim3(256), 0,
                               (hipStream_t)stream, sw, rows, heads, out, (long long)ldo);
            e = hipGetLastError();
            if (e != hipSuccess) return kea::fail((int)e, std::string("merge launch failed: ") + hipGetErrorString(e));
        }
        return KEA_OK;
    }
    const int nk = (int)((t + 63) / 64), kp = 64 * nk;
    const size_t lds = sizeof(float) * (size_t)(2 * kQB * head_dim + kQB * kp + (kQB - 1 + kp) * (head_dim + 4));
    if (!kea::fits_dispatch((t + kQB - 1) / kQB, 256)) return kea::fail(KEA_EINVAL, "too large for one launch");
    const dim3 grid((unsigned)((t + kQB - 1) / kQB), (unsigned)heads, (unsigned)batch);
    auto fn = nk == 1 ? relpos_attention_kernel<128, 1> : nk == 2 ? relpos_attention_kernel<128, 2>
            : nk == 3 ? relpos_attention_kernel<128, 3> : relpos_attention_kernel<128, 4>;
    if (lds > 65536) {
        hipError_t e = hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return kea::fail((int)e, std::string("LDS attribute refused: ") + hipGetErrorString(e));
    }
    hipLaunchKernelGGL(fn, grid, dim3(256), lds, (hipStream_t)stream, qkv, (long long)ld, pos, (long long)ldp, bias_u,
                       bias_v, out, (long long)ldo, (int)t, heads, scale);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return kea::fail((int)e, std::string("attention launch failed: ") + hipGetErrorString(e));
    return KEA_OK;
}

}  // namespace

extern "C" {

int kea_relpos_attention(const float *qkv, int64_t ld, const float *pos, int64_t ldp, const float *bias_u,
                         const float *bias_v, float *out, int64_t ldo, int64_t batch, int64_t t, int heads,
                         int head_dim, float scale, void *stream) {
    return attention(qkv, ld, pos, ldp, bias_u, bias_v, out, ldo, batch, t, heads, head_dim, scale, nullptr, 0,
                     stream);
}

int64_t kea_relpos_attention_workspace(int64_t batch, int64_t t, int heads) {
    if (batch < 1 || t < 1 || heads < 1 || !attention_splits(batch, t, heads)) return 0;
    return split_ws_bytes(batch, t, heads);
}

int kea_relpos_attention_ws(const float *qkv, int64_t ld, const float *pos, int64_t ldp, const float *bias_u,
                            const float *bias_v, float *out, int64_t ldo, int64_t batch, int64_t t, int heads,
                            int head_dim, float scale, void *workspace, int64_t workspace_bytes, void *stream) {
    return attention(qkv, ld, pos, ldp, bias_u, bias_v, out, ldo, batch, t, heads, head_dim, scale, workspace,
                     workspace_bytes, stream);
}

int kea_glu_dwconv(const float *x, int64_t ldx, const float *w, const float *bias, float *y, int64_t ldy,
                   int64_t batch, int64_t t, int64_t channels, int kernel, void *stream) {
    if (batch < 0 || t < 0 || channels < 1 || kernel < 1 || kernel % 2 == 0 || t > 65535 || batch > 65535)
        return kea::fail(KEA_EINVAL, "bad sizes (odd kernel width)");
    if (batch == 0 || t == 0) return KEA_OK;
    if (!x || !w || !y) return kea::fail(KEA_EINVAL, "null pointer");
    if (ldx < 2 * channels || ldy < channels) return kea::fail(KEA_EINVAL, "leading dimension too small");
    const dim3 grid((unsigned)((channels + 255) / 256), (unsigned)t, (unsigned)batch);
    hipLaunchKernelGGL(glu_dwconv_kernel, grid, dim3(256), 0, (hipStream_t)stream, x, (long long)ldx, w, bias, y,
                       (long long)ldy, (int)t, (int)channels, kernel);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return kea::fail((int)e, std::string("glu_dwconv launch failed: ") + hipGetErrorString(e));
    return KEA_OK;
}

int kea_subsample_front(const float *x, int64_t batch, int64_t t, int64_t f, const float *w1, const float *b1,
                        const float *w2, const float *b2, int64_t channels, float *y, void *stream) {
    if (batch < 0 || batch > 65535 || t < 1 || f < 1 || f > 128 || channels < 1 || channels > 65535 || t > INT32_MAX / 4)
        return kea::fail(KEA_EINVAL, "bad sizes (f <= 128)");
    if (batch == 0) return KEA_OK;
    if (!x || !w1 || !b1 || !w2 || !b2 || !y) return kea::fail(KEA_EINVAL, "null pointer");
    const int t1 = (int)((t - 1) / 2 + 1), f1 = (int)((f - 1) / 2 + 1);
    const int t2 = (t1 - 1) / 2 + 1, f2 = (f1 - 1) / 2 + 1;
    constexpr int CG = 32;
    const dim3 grid((unsigned)((t2 + kSubTT - 1) / kSubTT), (unsigned)((channels + CG - 1) / CG), (unsigned)batch);
    hipLaunchKernelGGL(subsample_front_kernel<CG>, grid, dim3(256), 0, (hipStream_t)stream, x, (int)t, (int)f, w1, b1,
                       w2, b2, y, (int)channels, t1, f1, t2, f2);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return kea::fail((int)e, std::string("subsample launch failed: ") + hipGetErrorString(e));
    return KEA_OK;
}

int kea_dwconv2d_s2(const float *x, const float *in_bias, const float *w, const float *bias, float *y, int64_t batch,
                    int64_t channels, int64_t h, int64_t wd, void *stream) {
    if (batch < 0 || channels < 1 || h < 1 || wd < 1 || batch * channels * h * wd > ((int64_t)1 << 40))
        return kea::fail(KEA_EINVAL, "bad sizes");
    if (batch == 0) return KEA_OK;
    if (!x || !w || !bias || !y) return kea::fail(KEA_EINVAL, "null pointer");
    const int h2 = (int)((h - 1) / 2 + 1), w2 = (int)((wd - 1) / 2 + 1);
    const long long total = batch * channels * (long long)h2 * w2;
    if (!kea::fits_dispatch((total + 255) / 256, 256)) return kea::fail(KEA_EINVAL, "too large for one launch");
    hipLaunchKernelGGL(dwconv_s2_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, (hipStream_t)stream, x,
                       in_bias, w, bias, y, (int)channels, (int)h, (int)wd, h2, w2, total);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return kea::fail((int)e, std::string("dwconv2d launch failed: ") + hipGetErrorString(e));
    return KEA_OK;
}

int kea_bias_relu_flatten(const float *x, const float *bias, float *y, int64_t batch, int64_t channels, int64_t h,
                          int64_t wd, void *stream) {
    if (batch < 0 || channels < 1 || h < 1 || wd < 1 || batch * channels * h * wd > ((int64_t)1 << 40))
        return kea::fail(KEA_EINVAL, "bad sizes");
    if (batch == 0) return KEA_OK;
    if (!x || !bias || !y) return kea::fail(KEA_EINVAL, "null pointer");
    const long long total = batch * channels * h * wd;
    if (!kea::fits_dispatch((total + 255) / 256, 256)) return kea::fail(KEA_EINVAL, "too large for one launch");
    hipLaunchKernelGGL(bias_relu_flatten_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, x, bias, y, (int)channels, (int)h, (int)wd, total);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return kea::fail((int)e, std::string("flatten launch failed: ") + hipGetErrorString(e));
    return KEA_OK;
}


int kea_logmel_normalize(const float *spec, int64_t batch, int64_t bins, int64_t frames, int64_t ld_t,
                         const float *fb, const int32_t *lo, const int32_t *hi, int64_t mels, float log_eps,
                         float std_eps, float *y, void *stream) {
    if (batch < 0 || batch > 65535 || bins < 1 || frames < 1 || ld_t < frames || mels < 1 || mels > 65535 ||
        bins * ld_t > ((int64_t)1 << 40))
        return kea::fail(KEA_EINVAL, "bad sizes");
    if (batch == 0) return KEA_OK;
    if (!spec || !fb || !lo || !hi || !y) return kea::fail(KEA_EINVAL, "null pointer");
    if ((uintptr_t)spec & 7) return kea::fail(KEA_EALIGN, "spec must be 8-byte aligned (interleaved complex)");
    hipLaunchKernelGGL(logmel_normalize_kernel, dim3((unsigned)mels, (unsigned)batch), dim3(256), 0,
                       (hipStream_t)stream, (const float2 *)spec, (int)bins, (int)frames, (long long)ld_t, fb, lo, hi,
                       (int)mels, log_eps, std_eps, y);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return kea::fail((int)e, std::string("logmel launch failed: ") + hipGetErrorString(e));
    return KEA_OK;
}

int kea_logmel_normalize_frames(const float *spec, int64_t batch, int64_t bins, int64_t frames, int64_t ld_f,
                                const float *fb, const int32_t *lo, const int32_t *hi, int64_t mels, float log_eps,
                                float std_eps, float *y, void *stream) {
    if (batch < 0 || batch > 65535 || bins < 1 || frames < 1 || ld_f < frames || mels < 1 || mels > 65535 ||
        bins * ld_f > ((int64_t)1 << 40))
        return kea::fail(KEA_EINVAL, "bad sizes");
    if (batch == 0) return KEA_OK;
    if (!spec || !fb || !lo || !hi || !y) return kea::fail(KEA_EINVAL, "null pointer");
    if ((uintptr_t)spec & 7) return kea::fail(KEA_EALIGN, "spec must be 8-byte aligned (interleaved complex)");
    hipLaunchKernelGGL(logmel_normalize_frames_kernel, dim3((unsigned)mels, (unsigned)batch), dim3(256), 0,
                       (hipStream_t)stream, (const float2 *)spec, (int)bins, (int)frames, (long long)ld_f, fb, lo, hi,
                       (int)mels, log_eps, std_eps, y);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return kea::fail((int)e, std::string("logmel launch failed: ") + hipGetErrorString(e));
    return KEA_OK;
}

int kea_stft_frames(const float *audio, int64_t batch, int64_t samples, float preemph, const float *window,
                    int64_t n_fft, int64_t hop, float *frames_out, void *stream) {
    if (batch < 0 || batch > 65535 || samples < 1 || n_fft < 2 || n_fft > 65536 || n_fft % 2 || hop < 1 ||
        samples > ((int64_t)1 << 40))
        return kea::fail(KEA_EINVAL, "bad sizes: batch in [0, 65535], samples >= 1, even n_fft in [2, 65536], hop >= 1");
    if (batch == 0) return KEA_OK;
    if (!audio || !window || !frames_out) return kea::fail(KEA_EINVAL, "null pointer");
    const int64_t frames = 1 + samples / hop, per_clip = frames * n_fft;
    const int64_t blocks = (per_clip + 255) / 256;
    if (blocks > 0x7fffffff) return kea::fail(KEA_EINVAL, "too many frames for one launch");
    hipLaunchKernelGGL(stft_frames_kernel, dim3((unsigned)blocks, (unsigned)batch), dim3(256), 0, (hipStream_t)stream,
                       audio, (long long)samples, preemph, window, (int)n_fft, (int)hop, (long long)frames, frames_out);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return kea::fail((int)e, std::string("stft frames launch failed: ") + hipGetErrorString(e));
    return KEA_OK;
}

}  // extern "C"
