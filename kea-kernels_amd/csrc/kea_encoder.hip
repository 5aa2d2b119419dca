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
#include "../../include/kea_encoder.h"

namespace {

constexpr int kQB = 8;        // query rows per workgroup
constexpr int kMaxT = 256;    // longest sequence a workgroup holds

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = v + __shfl_xor(v, off, 64);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

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

// Matrix-core form of the same attention for T <= 128 (one workgroup = 16 query rows of one (b, h), 4 waves), on
// v_mfma_f32_16x16x4_f32: lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16] per step and ends with
// D[4 (l / 16) + r][l % 16]. The head dimension is walked in the order d = 32 g + s (g = l / 16 the k lane group,
// s = 0..31 the step), so a lane's operand values are 32 contiguous floats (8 float4 loads straight from global
// memory); any order of the 128 terms is the same dot product up to FP32 rounding.
//   content scores   D = (q + u) K^T                      16 x 16 key tiles, waves over key tiles
//   position scores  D = (q + v) P_band^T                  the band of 16 + KP - 1 relative rows this block needs,
//                                                          taken back as bd[i][j] = band[i][j + 15 - i]
//   softmax          per row in LDS (exact two-pass, keys past T masked)
//   output           D = probs V over keys k = (KP/4) g + s, V transposed into LDS so operands are contiguous
template <int NKT>
__global__ void __launch_bounds__(256)
relpos_attention_mfma_kernel(const float *qkv, long long ld, const float *pos, long long ldp, const float *bias_u,
                             const float *bias_v, float *out, long long ldo, int T, int H, float scale) {
    constexpr int DK = 128, KP = 16 * NKT, NPT = NKT + 1, KS = KP / 4;
    constexpr int SP = KP + 4, BP = 16 * NPT + 4, VP = KP + 4;  // padded LDS row strides (floats)
    extern __shared__ __attribute__((aligned(16))) float sm[];
    float *Sc = sm, *Bd = Sc + 16 * SP, *Vt = Bd + 16 * BP;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, li = lane & 15, g = lane >> 4;
    const int b = blockIdx.z, h = blockIdx.y, i0 = blockIdx.x * 16;
    const float *qbase = qkv + (long long)b * T * ld + (long long)h * DK;
    const float *kbase = qbase + (long long)H * DK, *vbase = qbase + 2LL * H * DK;

    // V transposed into LDS: Vt[d][j] = V[j][d] (zero for j >= T); consecutive threads take consecutive keys
    for (int idx = tid; idx < KP * (DK / 4); idx += 256) {
        const int j = idx % KP, d = (idx / KP) * 4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (j < T) v = *(const float4 *)(vbase + (long long)j * ld + d);
        Vt[(d + 0) * VP + j] = v.x;
        Vt[(d + 1) * VP + j] = v.y;
        Vt[(d + 2) * VP + j] = v.z;
        Vt[(d + 3) * VP + j] = v.w;
    }

    // query operands with both position biases: row i0 + li, columns 32 g .. 32 g + 31
    float qa[32], qb[32];
    {
        const int t = i0 + li;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            float4 q = make_float4(0.f, 0.f, 0.f, 0.f);
            if (t < T) q = *(const float4 *)(qbase + (long long)t * ld + 32 * g + 4 * c);
            const float4 u = *(const float4 *)(bias_u + h * DK + 32 * g + 4 * c);
            const float4 v = *(const float4 *)(bias_v + h * DK + 32 * g + 4 * c);
            qa[4 * c] = q.x + u.x; qa[4 * c + 1] = q.y + u.y; qa[4 * c + 2] = q.z + u.z; qa[4 * c + 3] = q.w + u.w;
            qb[4 * c] = q.x + v.x; qb[4 * c + 1] = q.y + v.y; qb[4 * c + 2] = q.z + v.z; qb[4 * c + 3] = q.w + v.w;
        }
    }
    // one 16 x 16 tile of dot products: rows = the 16 queries, columns = 16 rows of `src` (zero where invalid)
    auto tile = [&](const float *q, const float *src, long long stride, int row, bool valid) {
        float kb[32];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (valid) v = *(const float4 *)(src + (long long)row * stride + 32 * g + 4 * c);
            kb[4 * c] = v.x; kb[4 * c + 1] = v.y; kb[4 * c + 2] = v.z; kb[4 * c + 3] = v.w;
        }
        v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < 32; ++st) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(q[st], kb[st], acc, 0, 0, 0);
        return acc;
    };
    for (int kt = wave; kt < NKT; kt += 4) {
        const int j = kt * 16 + li;
        const v4f acc = tile(qa, kbase, ld, j, j < T);
#pragma unroll
        for (int r = 0; r < 4; ++r) Sc[(4 * g + r) * SP + kt * 16 + li] = acc[r];
    }
    const int rbase = T - 1 - (i0 + 15);  // relative row of band position 0
    for (int pt = wave; pt < NPT; pt += 4) {
        const int r = rbase + pt * 16 + li;
        const v4f acc = tile(qb, pos + (long long)h * DK, ldp, r, r >= 0 && r <= 2 * T - 2);
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) Bd[(4 * g + rr) * BP + pt * 16 + li] = acc[rr];
    }
    __syncthreads();

    // softmax: wave w owns rows 4w .. 4w + 3; lane takes keys lane, lane + 64
    for (int i = 4 * wave; i < 4 * wave + 4; ++i) {
        float sv[2];
        float mx = -INFINITY;
#pragma unroll
        for (int n = 0; n < 2; ++n) {
            const int j = lane + 64 * n;
            sv[n] = -INFINITY;
            if (j < KP && j < T) sv[n] = (Sc[i * SP + j] + Bd[i * BP + j + 15 - i]) * scale;
            mx = fmaxf(mx, sv[n]);
        }
        mx = wave_max(mx);
        float sum = 0.f;
#pragma unroll
        for (int n = 0; n < 2; ++n) {
            sv[n] = expf(sv[n] - mx);
            sum = sum + sv[n];
        }
        const float inv = 1.0f / wave_sum(sum);
#pragma unroll
        for (int n = 0; n < 2; ++n) {
            const int j = lane + 64 * n;
            if (j < KP) Sc[i * SP + j] = sv[n] * inv;
        }
    }
    __syncthreads();

    // output: wave w computes head columns 32 w .. 32 w + 31 (two 16-column tiles)
    float pa[KS];
#pragma unroll
    for (int c = 0; c < KS; c += 4) {
        const float4 v = *(const float4 *)(Sc + li * SP + KS * g + c);
        pa[c] = v.x; pa[c + 1] = v.y; pa[c + 2] = v.z; pa[c + 3] = v.w;
    }
#pragma unroll
    for (int dt = 2 * wave; dt < 2 * wave + 2; ++dt) {
        v4f acc = {0.f, 0.f, 0.f, 0.f};
        const float *vrow = Vt + (dt * 16 + li) * VP + KS * g;
#pragma unroll
        for (int c = 0; c < KS; c += 4) {
            const float4 v = *(const float4 *)(vrow + c);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[c], v.x, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[c + 1], v.y, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[c + 2], v.z, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(pa[c + 3], v.w, acc, 0, 0, 0);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = i0 + 4 * g + r;
            if (t < T) out[((long long)b * T + t) * ldo + (long long)h * DK + dt * 16 + li] = acc[r];
        }
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

}  // namespace

extern "C" {

int kea_relpos_attention(const float *qkv, int64_t ld, const float *pos, int64_t ldp, const float *bias_u,
                         const float *bias_v, float *out, int64_t ldo, int64_t batch, int64_t t, int heads,
                         int head_dim, float scale, void *stream) {
    if (batch < 0 || t < 1 || heads < 1 || head_dim != 128)
        return kea::fail(KEA_EINVAL, "bad sizes (head_dim must be 128)");
    if (t > kMaxT) return kea::fail(KEA_EINVAL, "sequence longer than 256 frames: use the unfused attention");
    if (batch == 0) return KEA_OK;
    if (!qkv || !pos || !bias_u || !bias_v || !out) return kea::fail(KEA_EINVAL, "null pointer");
    if (ld < 3LL * heads * head_dim || ldp < (int64_t)heads * head_dim || ldo < (int64_t)heads * head_dim)
        return kea::fail(KEA_EINVAL, "leading dimension too small");
    if (((uintptr_t)qkv | (uintptr_t)pos | (uintptr_t)out | (uintptr_t)bias_u | (uintptr_t)bias_v) & 15 ||
        (ld | ldp | ldo) & 3)
        return kea::fail(KEA_EALIGN, "qkv, pos, out and the biases need 16-byte aligned rows");
    if (t <= 128) {
        const int nkt = (int)((t + 15) / 16), kp = 16 * nkt;
        const size_t lds = sizeof(float) * (size_t)(16 * (kp + 4) + 16 * (16 * (nkt + 1) + 4) + head_dim * (kp + 4));
        const dim3 grid((unsigned)((t + 15) / 16), (unsigned)heads, (unsigned)batch);
        void (*fn)(const float *, long long, const float *, long long, const float *, const float *, float *,
                   long long, int, int, float) = nullptr;
        switch (nkt) {
            case 1: fn = relpos_attention_mfma_kernel<1>; break;
            case 2: fn = relpos_attention_mfma_kernel<2>; break;
            case 3: fn = relpos_attention_mfma_kernel<3>; break;
            case 4: fn = relpos_attention_mfma_kernel<4>; break;
            case 5: fn = relpos_attention_mfma_kernel<5>; break;
            case 6: fn = relpos_attention_mfma_kernel<6>; break;
            case 7: fn = relpos_attention_mfma_kernel<7>; break;
            default: fn = relpos_attention_mfma_kernel<8>; break;
        }
        if (lds > 65536) {
            hipError_t e = hipFuncSetAttribute((const void *)fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) return kea::fail((int)e, std::string("LDS attribute refused: ") + hipGetErrorString(e));
        }
        hipLaunchKernelGGL(fn, grid, dim3(256), lds, (hipStream_t)stream, qkv, (long long)ld, pos, (long long)ldp,
                           bias_u, bias_v, out, (long long)ldo, (int)t, heads, scale);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return kea::fail((int)e, std::string("attention launch failed: ") + hipGetErrorString(e));
        return KEA_OK;
    }
    const int nk = (int)((t + 63) / 64), kp = 64 * nk;
    const size_t lds = sizeof(float) * (size_t)(2 * kQB * head_dim + kQB * kp + (kQB - 1 + kp) * (head_dim + 4));
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

}  // extern "C"
