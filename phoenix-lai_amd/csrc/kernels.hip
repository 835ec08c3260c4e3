// gfx950 kernels of the MoE FFN layer.  wave64 throughout; built with -ffp-contract=off so every
// float expression keeps the reference CPU path's rounding sequence (src/GemmaCpu.cs:376-422 over
// src/CpuRef*.cs): products and sums that the reference evaluates in a fixed order are evaluated
// in that order (per-row block chains, the router's dot chain, the rank-ordered combine), and the
// double-precision sums of squares of RmsNorm are reproduced through a certified error bound with
// an exact sequential fallback.
#include <algorithm>

#include "device_common.h"

namespace phx {

// ------------------------------------------------------------------------------ activation quantizers

// The integers of Q8_K super-block b of row `row` (lane l holds elements 4l..4l+3 packed in pk) stored in
// act's dot-product order (K4 / K6 / Q8K), with the sums of 16 (K4's s, and bh when set) and, with qh
// set, the matrix cores' fp16 copies; the block's scale is the caller's.  qrow is the wave's 64-dword
// LDS row through which the integers reach the packed orders.  Wave-level: all 64 lanes call it.
__device__ __forceinline__ void store_q8k_block(const Act& act, int64_t row, int b, int lane, uint32_t pk,
                                                uint32_t* qrow, float dval)
{
    int sm = (int)(int8_t)(pk & 0xFF) + (int)(int8_t)((pk >> 8) & 0xFF) + (int)(int8_t)((pk >> 16) & 0xFF) +
             (int)(int8_t)(pk >> 24);
    // block sums of 16: lanes 4j .. 4j + 3
    sm += dpp_i<0xb1>(sm, sm);  // 4-lane sum: quad swaps
    sm += dpp_i<0x4e>(sm, sm);
    if ((lane & 3) == 0) {
        if (act.fmt == ACT_K4 && act.s) act.s[row * act.sstride + b * 16 + (lane >> 2)] = sm;
        if (act.bh) act.bh[row * act.bhstride + b * 16 + (lane >> 2)] = (uint16_t)f2h_bits((float)sm);  // exact
    }
    if (act.fmt == ACT_Q8K) {
        if (act.q) ((uint32_t*)(act.q + row * act.qstride + (int64_t)b * 256))[lane] = pk;
        if (!act.qh) return;  // uniform
    }
    const uint8_t* qb = (const uint8_t*)qrow;
    qrow[lane] = pk;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    auto qv = [&](int e) { return (int)(int8_t)qb[e]; };
    if (!act.q) {  // uniform: only the matrix cores' copy is wanted
    } else if (act.fmt == ACT_K4) {  // dword (s, l) = x[32 s + l + 8 m], m = 0..3: lane = 8 s + l
        const int s8 = lane >> 3, l = lane & 7, e = 32 * s8 + l;
        ((uint32_t*)(act.q + row * act.qstride + (int64_t)b * 256))[lane] =
            (uint32_t)qb[e] | ((uint32_t)qb[e + 8] << 8) | ((uint32_t)qb[e + 16] << 16) | ((uint32_t)qb[e + 24] << 24);
    } else if (act.fmt == ACT_K6) {  // (P, l): lane = 8 P + l
        const int P = lane >> 3, l = lane & 7, e = 32 * P + l;
        uint32_t* dst = (uint32_t*)(act.q + row * act.qstride + (int64_t)b * 512);
        int* c = act.s + row * act.sstride + b * 128;
        dst[lane * 2 + 0] = (uint32_t)qb[e] | ((uint32_t)qb[e + 8] << 8);
        dst[lane * 2 + 1] = ((uint32_t)qb[e + 16] << 16) | ((uint32_t)qb[e + 24] << 24);
        c[(2 * P) * 8 + l] = -32 * (qv(e) + qv(e + 8));
        c[(2 * P + 1) * 8 + l] = -32 * (qv(e + 16) + qv(e + 24));
    }
    if (act.qh) {  // the matrix cores' copy: exact fp16 integers (or, folded, fp16 of q * dval), halves
                   // [l][s][mm']: lane = 8 l + s
        const int l = lane >> 3, s8 = lane & 7, e = 32 * s8 + l;
        uint32_t* hq = (uint32_t*)(act.qh + row * act.qhstride + (int64_t)b * 256) + l * 16 + s8 * 2;
        const float f = act.fold ? dval : 1.0f;
        hq[0] = f2h_bits((float)qv(e) * f) | (f2h_bits((float)qv(e + 16) * f) << 16);
        hq[1] = f2h_bits((float)qv(e + 8) * f) | (f2h_bits((float)qv(e + 24) * f) << 16);
    }
    // the row is rewritten by the wave's next block only after every lane's reads above
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Quantize one row (in LDS, `cols` floats) into format act, row index `row`.  Block-level (NT threads).
//  Q8_0: CpuRef.QuantizeQ8_0 (src/CpuRef.cs:49-62), plus the block sum of q for the Q4_0 offset.
//  K4/K6/Q8K: CpuRef.QuantizeQ8_K (src/CpuRefKQuants.cs:53-86), stored in the dot-product orders (and,
//  with qh / bh set, the matrix cores' fp16 copies).
template <int NT>
__device__ void quantize_row(const float* v, Act act, int64_t row)
{
    const int tid = threadIdx.x;
    if (act.fmt == ACT_Q8_0) {
        // eight lanes per 32-block, four values each (q8_0_oct); every thread runs the same number of
        // rounds (the shuffles need whole 8-lane groups), rounds past the last block store nothing
        const int nb = act.cols / 32, g = tid >> 3, l8 = tid & 7;
        for (int b0 = 0; b0 < nb; b0 += NT / 8) {
            const int b = b0 + g, bc = min(b, nb - 1);
            const float4 xv = *(const float4*)(v + bc * 32 + 4 * l8);
            float dval;
            int sum;
            const int qw = q8_0_oct(xv, &dval, &sum);
            if (b < nb) {
                if (act.q) ((int*)(act.q + row * act.qstride))[8 * b + l8] = qw;
                if (act.qh)  // the four integers as exact fp16, or folded with the block scale
                    *(uint2*)(act.qh + row * act.qhstride + 32 * b + 4 * l8) = act.fold ? fold_q4(qw, dval) : int_q4(qw);
                if (l8 == 0) {
                    act.d[row * act.dstride + b] = dval;
                    if (act.s) act.s[row * act.sstride + b] = sum;
                }
            }
        }
        return;
    }
    // Q8_K: one wave per 256-block, lane l holds elements 4l..4l+3; the block's integers pass through
    // the wave's LDS row to reach the packed orders
    __shared__ uint32_t qsm[NT / 64][64];
    const int nb = act.cols / 256, lane = tid & 63, wave = tid >> 6;
    for (int b = wave; b < nb; b += NT / 64) {
        const float4 v4 = ((const float4*)(v + b * 256))[lane];
        const float x[4] = {v4.x, v4.y, v4.z, v4.w};
        // the reference's scan: the first element of largest |x| (strict '>', from 0)
        float amax = 0.0f, vmax = 0.0f;
        int imax = 1 << 30;
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (fabsf(x[j]) > amax) {
                amax = fabsf(x[j]);
                vmax = x[j];
                imax = 4 * lane + j;
            }
        // the wave's first largest |x| by DPP steps (lanes outside a step's rows keep their own triple),
        // lane 63 ending with the result
        auto step = [&](auto C, auto RM) {
            constexpr int CTRL = decltype(C)::value, ROWMASK = decltype(RM)::value;
            const float oa = dpp_f<CTRL, ROWMASK>(amax, amax), ov = dpp_f<CTRL, ROWMASK>(vmax, vmax);
            const int oi = dpp_i<CTRL, ROWMASK>(imax, imax);
            if (oa > amax || (oa == amax && oi < imax)) {
                amax = oa;
                vmax = ov;
                imax = oi;
            }
        };
        step(ic<0xb1>{}, ic<0xf>{});
        step(ic<0x4e>{}, ic<0xf>{});
        step(ic<0x141>{}, ic<0xf>{});
        step(ic<0x140>{}, ic<0xf>{});
        step(ic<0x142>{}, ic<0xa>{});
        step(ic<0x143>{}, ic<0xc>{});
        amax = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(amax), 63));
        vmax = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(vmax), 63));
        const float iscale = amax == 0.0f ? 0.0f : -127.0f / vmax;
        int q[4];
#pragma unroll
        for (int j = 0; j < 4; j++) q[j] = amax == 0.0f ? 0 : min(nearest_int(iscale * x[j]), 127);
        const uint32_t pk = (uint32_t)(q[0] & 0xFF) | ((uint32_t)(q[1] & 0xFF) << 8) | ((uint32_t)(q[2] & 0xFF) << 16) |
                            ((uint32_t)q[3] << 24);
        const float dval = amax == 0.0f ? 0.0f : 1.0f / iscale;
        if (lane == 0) act.d[row * act.dstride + b] = dval;
        store_q8k_block(act, row, b, lane, pk, qsm[wave], dval);
    }
}

// ------------------------------------------------------------------------------ prologue
// Per token: the rms scale of x (shared by the router, pre_ffw_norm_2 and ffn_norm, which all
// normalise the same row: src/GemmaCpu.cs:386-389, :409, :349), the router input
// m = ((x * rinv) * (1/sqrt(d))) * s (src/GemmaCpu.cs:388-389), and the quantized expert input
// n = x * scale * pre_ffw_norm_2 (and the shared FFN input when the layer has one).
template <int NT>
__global__ __launch_bounds__(NT) void k_prologue(int d, float eps, const float* __restrict__ x,
                                                 const float* __restrict__ gis, const float* __restrict__ pre2,
                                                 const float* __restrict__ ffn_norm, float* __restrict__ router_in,
                                                 float* __restrict__ xscale, Act act_gu, Act act_sh, int* flags)
{
    extern __shared__ __align__(16) float sbuf[];
    __shared__ double red[NT];
    const int t = blockIdx.x, tid = threadIdx.x;
    TL_STAMP(0, 0, 0);
    const float* xr = x + (int64_t)t * d;
    float scale = rms_scale_from_mean(mean_sq_cert<NT>(xr, d, red, flags), eps);
    TL_STAMP(0, 0, 1);
    float sc = 1.0f / (float)__dsqrt_rn((double)d);
    // four values per thread and round (d and the activation widths are multiples of 32)
    const float4* x4 = (const float4*)xr;
    auto fill = [&](const float* nw, int cols) {
        for (int i4 = tid; i4 < cols / 4; i4 += NT) {
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (4 * i4 < d) {
                const float4 xv = x4[i4], nv = ((const float4*)nw)[i4];
                v = make_float4(xv.x * scale * nv.x, xv.y * scale * nv.y, xv.z * scale * nv.z, xv.w * scale * nv.w);
            }
            ((float4*)sbuf)[i4] = v;
        }
    };
    if (router_in) {  // uniform; null where the router forms m from x and the scale itself
        float* ri = router_in + (int64_t)t * d;
        for (int i4 = tid; i4 < d / 4; i4 += NT) {
            const float4 xv = x4[i4], gv = ((const float4*)gis)[i4];
            ((float4*)ri)[i4] = make_float4(xv.x * scale * sc * gv.x, xv.y * scale * sc * gv.y,
                                            xv.z * scale * sc * gv.z, xv.w * scale * sc * gv.w);
        }
    }
    fill(pre2, act_gu.cols);
    __syncthreads();
    TL_STAMP(0, 0, 2);
    quantize_row<NT>(sbuf, act_gu, t);
    TL_STAMP(0, 0, 3);
    if (ffn_norm) {
        __syncthreads();
        fill(ffn_norm, act_sh.cols);
        __syncthreads();
        quantize_row<NT>(sbuf, act_sh, t);
    }
    if (tid == 0) xscale[t] = scale;
    TL_STAMP(0, 0, 4);
}

// The same with the row held in registers (Q float4 per thread, rows up to 4 Q NT columns): x is read
// from memory once, for the mean of squares and for every normed copy.
template <int NT, int Q>
__global__ __launch_bounds__(NT) void k_prologue_r(int d, float eps, const float* __restrict__ x,
                                                   const float* __restrict__ gis, const float* __restrict__ pre2,
                                                   const float* __restrict__ ffn_norm, float* __restrict__ router_in,
                                                   float* __restrict__ xscale, Act act_gu, Act act_sh, int* flags)
{
    extern __shared__ __align__(16) float sbuf[];
    __shared__ double red[NT / 64 + 1];
    const int t = blockIdx.x, tid = threadIdx.x, n4 = d / 4;
    TL_STAMP(0, 0, 0);
    const float* xr = x + (int64_t)t * d;
    const float4* x4 = (const float4*)xr;
    const float4 z4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    float4 xv[Q], pv[Q];  // the row and the pre_ffw_norm_2 weights, both loaded at once
#pragma unroll
    for (int q = 0; q < Q; q++) {
        const int i4 = tid + q * NT;
        xv[q] = i4 < n4 ? x4[i4] : z4;
        pv[q] = i4 < n4 ? ((const float4*)pre2)[i4] : z4;
    }
    double s2 = 0.0;  // this thread's squares (at most 4 Q of them), any order: the bound covers it
#pragma unroll
    for (int q = 0; q < Q; q++) {
        s2 += (double)xv[q].x * (double)xv[q].x;
        s2 += (double)xv[q].y * (double)xv[q].y;
        s2 += (double)xv[q].z * (double)xv[q].z;
        s2 += (double)xv[q].w * (double)xv[q].w;
    }
    const float scale = rms_scale_from_mean(mean_sq_cert_from<NT>(s2, 4 * Q, xr, d, red, flags), eps);
    TL_STAMP(0, 0, 1);
    const float sc = 1.0f / (float)__dsqrt_rn((double)d);
    if (router_in) {  // uniform; null where the router forms m from x and the scale itself
        float4* ri = (float4*)(router_in + (int64_t)t * d);
#pragma unroll
        for (int q = 0; q < Q; q++) {
            const int i4 = tid + q * NT;
            if (i4 < n4) {
                const float4 xq = xv[q], gv = ((const float4*)gis)[i4];
                ri[i4] = make_float4(xq.x * scale * sc * gv.x, xq.y * scale * sc * gv.y, xq.z * scale * sc * gv.z,
                                     xq.w * scale * sc * gv.w);
            }
        }
    }
    auto fill = [&](const float* nw, int cols) {  // nw null: pre_ffw_norm_2 from registers
#pragma unroll
        for (int q = 0; q < Q; q++) {
            const int i4 = tid + q * NT;
            if (i4 < cols / 4) {
                float4 v = z4;
                if (i4 < n4) {
                    const float4 xq = xv[q], nv = nw ? ((const float4*)nw)[i4] : pv[q];
                    v = make_float4(xq.x * scale * nv.x, xq.y * scale * nv.y, xq.z * scale * nv.z, xq.w * scale * nv.w);
                }
                ((float4*)sbuf)[i4] = v;
            }
        }
    };
    fill(nullptr, act_gu.cols);
    __syncthreads();
    TL_STAMP(0, 0, 2);
    quantize_row<NT>(sbuf, act_gu, t);
    TL_STAMP(0, 0, 3);
    if (ffn_norm) {
        __syncthreads();
        fill(ffn_norm, act_sh.cols);
        __syncthreads();
        quantize_row<NT>(sbuf, act_sh, t);
    }
    if (tid == 0) xscale[t] = scale;
    TL_STAMP(0, 0, 4);
}

void launch_prologue(hipStream_t st, int T, int d, float eps, const float* x, const float* gis, const float* pre2,
                     const float* ffn_norm, float* router_in, float* xscale, Act act_gu, Act act_sh, int* flags)
{
    int cols = act_gu.cols > act_sh.cols ? act_gu.cols : act_sh.cols;
    if (cols < d) cols = d;
    // rows of more than 3072 columns: a thread per four columns (one load round per phase, the Q8_K
    // super-blocks one per wave; measured faster at C4's 4096, slower at C3's 2816 where the launch is
    // bound by HBM with 256)
    const size_t lds = (size_t)cols * sizeof(float);
#define PRO_R(NT, Q) \
    launch(k_prologue_r<NT, Q>, dim3(T), dim3(NT), lds, st, d, eps, x, gis, pre2, ffn_norm, router_in, xscale, act_gu, \
           act_sh, flags)
    const int c4 = cols / 4;
    if (c4 > 768) {
        switch ((c4 + 1023) / 1024) {
        case 1: PRO_R(1024, 1); return;
        case 2: PRO_R(1024, 2); return;
        case 3: PRO_R(1024, 3); return;
        case 4: PRO_R(1024, 4); return;
        default: break;  // wider rows: the kernel that reads them twice
        }
    } else {
        switch ((c4 + 255) / 256) {
        case 1: PRO_R(256, 1); return;
        case 2: PRO_R(256, 2); return;
        default: PRO_R(256, 3); return;
        }
    }
#undef PRO_R
    if (cols / 4 > 768)
        launch(k_prologue<1024>, dim3(T), dim3(1024), lds, st, d, eps, x, gis, pre2, ffn_norm, router_in, xscale, act_gu,
               act_sh, flags);
    else
        launch(k_prologue<256>, dim3(T), dim3(256), lds, st, d, eps, x, gis, pre2, ffn_norm, router_in, xscale, act_gu,
               act_sh, flags);
}

// ------------------------------------------------------------------------------ top-k and weights
// One wave per token (topk_wave: lane e + 64 q holds expert e + 64 q's logit in v[q], avail[q] whether
// the expert exists; lanes j < k write rank j's id and weight to ids[j], wout[j]), in k_topk or, where
// one router workgroup holds every expert (E <= 64), at the end of the router kernel.  k rounds of the
// reference's scan (GemmaCpu.cs:400-405, see scan_start): the
// lowest-index untaken expert when its logit is NaN, else the argmax of the untaken non-NaN logits
// with the lower expert index winning ties (the rank rule of KernelsMoe.RouterSelect,
// src/KernelsMoe.cs:64-78, for NaN-free logits).
// Weights as GemmaCpu.cs:406-407,417: p_j = (float)exp((double)(l_j - l_0)), sum in double,
// w_j = (float)(p_j / sum) * down_scale[e_j]; rule 1 keeps the CPU's in-place sel[0] update.
__device__ __forceinline__ void topk_wave(const float (&v)[4], bool (&avail)[4], int k, int rule,
                                          const float* __restrict__ ds, int* __restrict__ ids,
                                          float* __restrict__ wout)
{
    const int lane = threadIdx.x & 63;
    float my_sel = 0.0f;
    int my_id = 0;
    float dsv[4];  // the down scales, loaded now: their latency hides behind the rounds
#pragma unroll
    for (int q = 0; q < 4; q++) dsv[q] = avail[q] ? ds[lane + 64 * q] : 0.0f;
    for (int j = 0; j < k; j++) {
        bool e0_nan;
        const int e0 = scan_start(avail, v, &e0_nan);
        int bi;
        if (e0_nan) {  // uniform: the scan keeps e0
            bi = e0;
        } else {
            // the round's maximum as one 64-bit key per lane: the logit's order-preserving bits above
            // (both zeros as +0, which compare equal), the complemented index below (ties to the lower
            // index); a NaN or taken expert's key is 0, below every number's
            unsigned bh = 0u, bl = 0u;
#pragma unroll
            for (int q = 0; q < 4; q++)
                if (avail[q] && v[q] == v[q]) {
                    const unsigned kh = sortable_f32(v[q] == 0.0f ? 0.0f : v[q]), kl = ~(unsigned)(lane + 64 * q);
                    if (kh > bh || (kh == bh && kl > bl)) {
                        bh = kh;
                        bl = kl;
                    }
                }
            wave_max_key(bh, bl);
            bi = bh ? (int)~bl : -1;  // -1: no expert left (every lane agrees)
        }
        if (bi >= 0 && lane == (bi & 63)) avail[bi >> 6] = false;
        // the round's logit, from the lane that holds it (bi is wave-uniform)
        const int q0 = bi < 0 ? 0 : bi >> 6;
        const float vq = q0 == 0 ? v[0] : q0 == 1 ? v[1] : q0 == 2 ? v[2] : v[3];
        const float bv = bi < 0 ? 0.0f : __int_as_float(__builtin_amdgcn_readlane(__float_as_int(vq), bi & 63));
        if (lane == j) {  // lane j keeps rank j
            my_sel = bv;
            my_id = bi < 0 ? 0 : bi;
        }
    }
    // weights (src/GemmaCpu.cs:406-407,417), lane j for rank j: p_j = (float)exp((double)(l_j - top)),
    // the double sum in rank order, w_j = (float)(p_j / sum) * down_scale; GemmaCpu.cs:407 overwrites
    // sel[0] with p_0 = exp(0) = 1 before the later terms read it (rule 1)
    const float sel0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(my_sel), 0));
    const float top = (rule == 1 && lane > 0) ? 1.0f : sel0;
    const float pj = lane < k ? (float)exp((double)(my_sel - top)) : 0.0f;
    double sum = 0.0;
    for (int q = 0; q < k; q++) sum += (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(pj), q));
    // ds[my_id] from the lane that loaded it (every lane takes part in the exchanges)
    float dj = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const float t = __shfl(dsv[q], my_id & 63, 64);
        if ((my_id >> 6) == q) dj = t;
    }
    if (lane < k) {
        ids[lane] = my_id;
        wout[lane] = (float)((double)pj / sum) * dj;
    }
}

// the top-k of token t in a router wave whose lane e holds expert e's logit s (E <= 64)
__device__ __forceinline__ void topk_row(const TopkOut& to, int t, float s, bool valid)
{
    const float v[4] = {s, 0.0f, 0.0f, 0.0f};
    bool avail[4] = {valid, false, false, false};
    topk_wave(v, avail, to.k, to.rule, to.ds, to.ids + (int64_t)t * to.k, to.w + (int64_t)t * to.k);
}

// ------------------------------------------------------------------------------ router logits
// logits[t][e] = sum_i W[e][i] * m[t][i] as the sequential float sum of GemmaCpu.cs:393-394: one lane
// per (t, e), the products rounded, then added in index order.  W is stored [d/4][E][4] so the 64
// lanes (experts) of a wave read 1 KB contiguous; m is wave-uniform.
template <int TB>
__global__ __launch_bounds__(64) void k_router_exact(int T, int d, int E, const float4* __restrict__ wt4,
                                                     const float* __restrict__ rin, float* __restrict__ logits,
                                                     TopkOut to)
{
    extern __shared__ float4 srin[];  // [TB][d / 4]: the wave's token rows of m
    const int lane = threadIdx.x, e = blockIdx.x * 64 + lane, t0 = blockIdx.y * TB;
    const int ee = e < E ? e : E - 1;
    const float4* w = wt4 + ee;
    const int n4 = d / 4;  // d % 32 == 0
    for (int j = 0; j < TB; j++) {
        const float4* m = (const float4*)(rin + (int64_t)min(t0 + j, T - 1) * d);
        for (int i = lane; i < n4; i += 64) srin[j * n4 + i] = m[i];
    }
    float4 wv[8];
#pragma unroll
    for (int q = 0; q < 8; q++) wv[q] = w[(int64_t)q * E];
    __syncthreads();
    float s[TB];
#pragma unroll
    for (int j = 0; j < TB; j++) s[j] = 0.0f;
    for (int i = 0; i < n4; i += 8) {
        float4 wn[8];
#pragma unroll
        for (int q = 0; q < 8; q++) wn[q] = w[(int64_t)min(i + 8 + q, n4 - 1) * E];  // the next chunk (clamped)
#pragma unroll
        for (int q = 0; q < 8; q++) {
#pragma unroll
            for (int j = 0; j < TB; j++) {
                const float4 mv = srin[j * n4 + i + q];  // one LDS broadcast for the wave
                s[j] += wv[q].x * mv.x;
                s[j] += wv[q].y * mv.y;
                s[j] += wv[q].z * mv.z;
                s[j] += wv[q].w * mv.w;
            }
        }
#pragma unroll
        for (int q = 0; q < 8; q++) wv[q] = wn[q];
    }
    if (e < E) {
#pragma unroll
        for (int j = 0; j < TB; j++)
            if (t0 + j < T) logits[(int64_t)(t0 + j) * E + e] = s[j];
    }
    if (to.ids) {  // uniform: every expert is in this wave (E <= 64)
#pragma unroll
        for (int j = 0; j < TB; j++)
            if (t0 + j < T) topk_row(to, t0 + j, s[j], e < E);
    }
}

// Many tokens: a workgroup of four waves takes 64 experts and 4 TPW tokens; wave w carries tokens
// TPW w .. TPW w + TPW - 1, lane e expert e, each chain in index order (the reference's sequential
// sum).  The router columns of the 64 experts and the token rows of m stream through LDS in
// 128-element chunks (two buffers): every thread loads its share of the next chunk into registers
// before the current chunk's adds and stores it after, one barrier per chunk.  W leaves L2 once per
// 4 TPW tokens and reaches the lanes at the LDS rate, and with every operand read from LDS the reads
// of the next eight columns can go out ahead of the current eight's adds (LDS reads complete in
// order).  TPW 2 halves W's traffic, TPW 1 doubles the waves (for fewer tokens).
constexpr int RXW_CH4 = 32;  // float4 columns per chunk
template <int TPW>
__global__ __launch_bounds__(256, 2) void k_router_exact_wide(int T, int d, int E, const float4* __restrict__ wt4,
                                                              const float* __restrict__ rin,
                                                              float* __restrict__ logits, TopkOut to, RouterX rx)
{
    constexpr int TOK = 4 * TPW;
    __shared__ float4 wbuf[2][RXW_CH4][64];
    __shared__ float4 mbuf[2][TOK][RXW_CH4];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int e0 = blockIdx.x * 64, e = e0 + lane;
    const int tb = blockIdx.y * TOK, t0 = tb + TPW * wave;
    const int n4 = d / 4, nch = (n4 + RXW_CH4 - 1) / RXW_CH4;
    // this thread's share of a chunk: W columns (tid / 64) + 4 k, k = 0..7, of expert e0 + lane, and
    // (threads below 32 TOK) column tid % 32 of token row tid / 32
    const int er = min(e, E - 1), cr = tid >> 6, mt = min(tid >> 5, TOK - 1), mc = tid & 31;
    const bool mld = tid < 32 * TOK;
    const int mtok = min(tb + mt, T - 1);
    const float4* mrow = (const float4*)(rin + (int64_t)mtok * d);
    // rx.xscale set: rin is x and m = ((x * rinv) * (1/sqrt(d))) * s is formed here as the prologue would
    // (src/GemmaCpu.cs:388-389), the row's rms scale rinv from the prologue
    const float rinv = rx.xscale ? rx.xscale[mtok] : 0.0f, sc = 1.0f / (float)__dsqrt_rn((double)d);
    const float4* gis4 = (const float4*)(rx.xscale ? rx.gis : rin);
    // the loads go out with the chunk's others; m is formed where it is stored, after the chunk's adds
    auto mval = [&](const float4& v, const float4& gv) {
        return rx.xscale ? make_float4(v.x * rinv * sc * gv.x, v.y * rinv * sc * gv.y, v.z * rinv * sc * gv.z,
                                       v.w * rinv * sc * gv.w)
                         : v;
    };
    float4 st[8], sm, sg;
#pragma unroll
    for (int k = 0; k < 8; k++) st[k] = wt4[(int64_t)min(cr + 4 * k, n4 - 1) * E + er];
    sm = mrow[min(mc, n4 - 1)];
    sg = gis4[min(mc, n4 - 1)];
#pragma unroll
    for (int k = 0; k < 8; k++) wbuf[0][cr + 4 * k][lane] = st[k];
    if (mld) mbuf[0][mt][mc] = mval(sm, sg);
    __syncthreads();
    float s[TPW];
#pragma unroll
    for (int j = 0; j < TPW; j++) s[j] = 0.0f;
    for (int c = 0; c < nch; c++) {
        const int buf = c & 1;
        // the next chunk's loads (past the last chunk: a clamped reload nobody reads)
        const int cn = min(c + 1, nch - 1) * RXW_CH4;
#pragma unroll
        for (int k = 0; k < 8; k++) st[k] = wt4[(int64_t)min(cn + cr + 4 * k, n4 - 1) * E + er];
        sm = mrow[min(cn + mc, n4 - 1)];
        sg = gis4[min(cn + mc, n4 - 1)];
        const int ni = min(RXW_CH4, n4 - c * RXW_CH4);  // d % 32 == 0: ni % 8 == 0
#pragma unroll 8
        for (int i = 0; i < ni; i++) {
            const float4 w = wbuf[buf][i][lane];
            float4 a[TPW];
#pragma unroll
            for (int j = 0; j < TPW; j++) a[j] = mbuf[buf][TPW * wave + j][i];
#pragma unroll
            for (int j = 0; j < TPW; j++) s[j] += w.x * a[j].x;
#pragma unroll
            for (int j = 0; j < TPW; j++) s[j] += w.y * a[j].y;
#pragma unroll
            for (int j = 0; j < TPW; j++) s[j] += w.z * a[j].z;
#pragma unroll
            for (int j = 0; j < TPW; j++) s[j] += w.w * a[j].w;
        }
#pragma unroll
        for (int k = 0; k < 8; k++) wbuf[buf ^ 1][cr + 4 * k][lane] = st[k];  // read before the last barrier
        if (mld) mbuf[buf ^ 1][mt][mc] = mval(sm, sg);
        __syncthreads();
    }
    if (e < E) {
#pragma unroll
        for (int j = 0; j < TPW; j++)
            if (t0 + j < T) logits[(int64_t)(t0 + j) * E + e] = s[j];
    }
    if (to.ids) {  // uniform: every expert is in this workgroup (E <= 64), the wave's tokens are its own
#pragma unroll
        for (int j = 0; j < TPW; j++)
            if (t0 + j < T) topk_row(to, t0 + j, s[j], e < E);
    }
}

// Fewer tokens (latency-bound: too few chains to hide the loads): a workgroup of NWV waves takes 64
// experts and NWV tokens (one per wave), with the router columns streamed through a ring of RR_RING
// LDS slots by direct global -> LDS loads, RR_RING - 1 chunks of 64 elements ahead: a wave issues
// 16 / NWV 1-KB column loads (the 64 experts of one float4 column are contiguous) and its token's 16
// float4 of m per chunk, so its own count of outstanding loads tells when a chunk has landed.  One wave
// alone issues a VALU instruction about every 8.7 cycles and two or more waves share a SIMD at about 3
// (measured on MI355X), so with 32 or more token groups eight waves per workgroup (two per SIMD) run
// the chains faster than four.
constexpr int RR_CH4 = 16, RR_RING = 4;
template <int NWV>
__global__ __launch_bounds__(64 * NWV) void k_router_ring(int T, int d, int E, const float4* __restrict__ wt4,
                                                          const float* __restrict__ rin, float* __restrict__ logits,
                                                          TopkOut to)
{
    constexpr int CPW = RR_CH4 / NWV, DMA = CPW + 1;  // columns and direct loads per wave and chunk
    __shared__ float4 wring[RR_RING][RR_CH4][64];
    __shared__ float4 mring[RR_RING][NWV][RR_CH4];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int e = blockIdx.x * 64 + lane, t = blockIdx.y * NWV + wave;
    const int n4 = d / 4, nch = (n4 + RR_CH4 - 1) / RR_CH4;  // d % 64 == 0: whole chunks
    const float4* wsrc = wt4 + min(e, E - 1);                      // column c: + c * E
    const float4* msrc = (const float4*)(rin + (int64_t)min(t, T - 1) * d) + min(lane, RR_CH4 - 1);
    auto issue = [&](int c) {  // chunk c (clamped: past the end a harmless reload) into its slot
        const int cc = min(c, nch - 1), slot = c % RR_RING;
#pragma unroll
        for (int j = 0; j < CPW; j++)
            __builtin_amdgcn_global_load_lds((glb_void_t)(wsrc + (int64_t)(cc * RR_CH4 + CPW * wave + j) * E),
                                             (lds_void_t)&wring[slot][CPW * wave + j][0], 16, 0, 0);
        if (lane < RR_CH4)
            __builtin_amdgcn_global_load_lds((glb_void_t)(msrc + cc * RR_CH4), (lds_void_t)&mring[slot][wave][0], 16, 0, 0);
    };
#pragma unroll
    for (int c = 0; c < RR_RING - 1; c++) issue(c);
    float s = 0.0f;
    const uint32_t w0 = (uint32_t)(uintptr_t)(lds_void_t)&wring[0][0][lane];
    const uint32_t m0 = (uint32_t)(uintptr_t)(lds_void_t)&mring[0][wave][0];
    for (int c = 0; c < nch; c++) {
        // chunk c has landed once at most the two later chunks' loads are outstanding; the barrier then
        // publishes it and ends every wave's reads of the slot that issue(c + RING - 1) refills
        __builtin_amdgcn_s_waitcnt((DMA * (RR_RING - 2)) | (0x7 << 4) | (0xF << 8));
        __builtin_amdgcn_s_barrier();
        issue(c + RR_RING - 1);
        const int slot = c % RR_RING;
        // explicit reads (see device_common.h), four columns per batch, the next batch's reads issued
        // before this batch's adds
        const uint32_t wa = w0 + slot * (RR_CH4 * 64 * 16), ma = m0 + slot * (NWV * RR_CH4 * 16);
        u32x4 W[2][4], M[2][4];
        auto reads = [&](auto GC) {
            constexpr int g = decltype(GC)::value, b = g & 1;
            W[b][0] = ds_r128<(4 * g + 0) * 1024>(wa);
            W[b][1] = ds_r128<(4 * g + 1) * 1024>(wa);
            W[b][2] = ds_r128<(4 * g + 2) * 1024>(wa);
            W[b][3] = ds_r128<(4 * g + 3) * 1024>(wa);
            M[b][0] = ds_r128<(4 * g + 0) * 16>(ma);  // one LDS broadcast for the wave
            M[b][1] = ds_r128<(4 * g + 1) * 16>(ma);
            M[b][2] = ds_r128<(4 * g + 2) * 16>(ma);
            M[b][3] = ds_r128<(4 * g + 3) * 16>(ma);
        };
        auto landed = [&](int b) {
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int j = 0; j < 4; j++) {
                tie(W[b][j]);
                tie(M[b][j]);
            }
        };
        auto adds = [&](int b) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const float4 w = __builtin_bit_cast(float4, W[b][j]), m = __builtin_bit_cast(float4, M[b][j]);
                s += w.x * m.x;
                s += w.y * m.y;
                s += w.z * m.z;
                s += w.w * m.w;
            }
        };
        reads(ic<0>{});
        landed(0);
        reads(ic<1>{});
        adds(0);
        landed(1);
        reads(ic<2>{});
        adds(1);
        landed(0);
        reads(ic<3>{});
        adds(0);
        landed(1);
        adds(1);
    }
    __builtin_amdgcn_s_waitcnt(0);  // the reloads past the last chunk land before the workgroup ends
    if (e < E && t < T) logits[(int64_t)t * E + e] = s;
    if (to.ids && t < T) topk_row(to, t, s, e < E);  // uniform: every expert is in this wave (E <= 64)
}

// Eight tokens per workgroup where that still makes 1024 workgroups (enough chains to keep the SIMDs
// busy: compute-bound), else four with the deeper load ring (d % 64 == 0), else one wave per (64
// experts, token) with the token's row of m in LDS.
bool router_reads_x(int T, int d, int E) { return T * ((E + 63) / 64) >= 1024; }

void launch_router_exact(hipStream_t st, int T, int d, int E, const float* wt4, const float* rin, float* logits,
                         TopkOut to, RouterX rx)
{
    const int gx = (E + 63) / 64;
    if (gx > 1) to.ids = nullptr;  // the top-k needs every expert of a token in one wave
    const float4* w = (const float4*)wt4;
    if (T * gx >= 1024)
        launch(k_router_exact_wide<2>, dim3(gx, (T + 7) / 8), dim3(256), 0, st, T, d, E, w, rin, logits, to, rx);
    else if (d % 64 == 0 && (T + 7) / 8 * gx >= 32)
        launch(k_router_ring<8>, dim3(gx, (T + 7) / 8), dim3(512), 0, st, T, d, E, w, rin, logits, to);
    else if (d % 64 == 0)
        launch(k_router_ring<4>, dim3(gx, (T + 3) / 4), dim3(256), 0, st, T, d, E, w, rin, logits, to);
    else
        launch(k_router_exact<1>, dim3(gx, T), dim3(64), (uint32_t)(d * 4), st, T, d, E, w, rin, logits, to);
}

__global__ __launch_bounds__(64) void k_topk(int E, int k, int rule, const float* __restrict__ logits,
                                             const float* __restrict__ ds, int* __restrict__ ids, float* __restrict__ wout)
{
    const int t = blockIdx.x, lane = threadIdx.x;
    float v[4];
    bool avail[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        int e = lane + 64 * q;
        avail[q] = e < E;
        v[q] = avail[q] ? logits[(int64_t)t * E + e] : 0.0f;
    }
    topk_wave(v, avail, k, rule, ds, ids + (int64_t)t * k, wout + (int64_t)t * k);
}

void launch_topk(hipStream_t st, int T, int E, int k, int rule, const float* logits, const float* ds, int* ids, float* w)
{
    launch(k_topk, dim3(T), dim3(64), 0, st, E, k, rule, logits, ds, ids, w);
}

// ------------------------------------------------------------------------------ dispatch
// Per-expert ascending assignment lists (the lists of KernelsMoe.Bucket, src/KernelsMoe.cs:281-330)
// as one stable counting sort, and the work list of (expert, first list position, count <= A) tiles
// for the grouped kernels.
// Workgroups of 16 waves, one per chunk of 1024 assignments (2048 measured 0.7 µs slower at C3); wave w
// owns the contiguous segment w of the chunk and walks it 64 at a time.  In a batch, eight ballots over the expert-id bits give each
// lane the mask of the lanes holding the same expert: its rank among them (a popcount of the lower
// lanes) and their count, so no lane waits on another.  Every workgroup counts each expert over the
// whole list and before its chunk, and each segment's experts; a prefix over the experts gives the
// list offsets, the counts before the chunk and over the earlier segments each segment's start in
// every list, and a last pass places the chunk's assignments: the lists come out in ascending
// assignment order (a stable counting sort, the lists of KernelsMoe.Bucket).
constexpr int DSP_NT = 1024, DSP_SEG = DSP_NT / 64, DSP_CH = 1024;

__device__ __forceinline__ uint64_t same_expert_mask(int e, bool valid, int nbits)
{
    uint64_t m = __ballot(valid);
    for (int b = 0; b < nbits; b++) {
        const bool bit = (e >> b) & 1;
        const uint64_t v = __ballot(bit);
        m &= bit ? v : ~v;
    }
    return valid ? m : 0ull;
}

// Workgroup g places the assignments of chunk g, [g CH, (g + 1) CH).  Every workgroup reads the whole id
// list (the previous launch wrote it: one cold read, L2 hits after) and counts, per expert, the
// assignments of the list and those before its chunk, so the placements of the chunks need no exchange
// between workgroups: assignment a of expert e lands at offsets[e] + (e's assignments before the chunk) +
// (e's assignments before a in the chunk), ascending a within each expert.  Workgroup 0 also writes the
// offsets, the tile count and the tiles.
__global__ __launch_bounds__(DSP_NT) void k_dispatch(int n, int E, int A, const int* __restrict__ ids,
                                                     int* __restrict__ offsets, int* __restrict__ perm,
                                                     Tile* __restrict__ tiles, int* __restrict__ ntiles)
{
    __shared__ int cnt[DSP_SEG][PHX_MAX_EXPERTS_DEV];
    __shared__ int pre[PHX_MAX_EXPERTS_DEV], tot[PHX_MAX_EXPERTS_DEV];
    __shared__ int toff[PHX_MAX_EXPERTS_DEV + 1], tb[PHX_MAX_EXPERTS_DEV + 1];
    __shared__ int wsum[2][DSP_SEG], tsum[5][DSP_SEG];
    extern __shared__ uint8_t sid[];  // the expert ids as bytes [n]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c0 = blockIdx.x * DSP_CH, c1 = min(n, c0 + DSP_CH);  // this workgroup's chunk (c0 % 64 == 0)
    int nbits = 0;
    while ((1 << nbits) < E) nbits++;
    // the ids in batches of 16 loads per thread (the first batch goes out before the counters are cleared)
    int v[16];
    auto load = [&](int i0) {
#pragma unroll
        for (int u = 0; u < 16; u++) v[u] = ids[min(i0 + DSP_NT * u, n - 1)];
    };
    load(tid);
    for (int i = tid; i < DSP_SEG * PHX_MAX_EXPERTS_DEV; i += DSP_NT) (&cnt[0][0])[i] = 0;
    for (int i = tid; i < PHX_MAX_EXPERTS_DEV; i += DSP_NT) {
        pre[i] = 0;
        tot[i] = 0;
    }
    const bool multi = gridDim.x > 1;  // uniform
    const int nwe = (E + 63) >> 6;     // the waves whose threads hold experts (one per thread below)
    __syncthreads();
    // with several chunks, counts over the list as the ids arrive: every lane adds its assignment into its
    // wave's own row by an LDS atomic (the list total in the low 16 bits, the count before the chunk in
    // the high 16, n <= 65535), summed per expert below (one workgroup: its segments cover the list); then
    // per segment of the chunk.  (A rank-free count needs no same-expert mask: its eight ballots per
    // batch made this pass VALU-bound, 256 batches of ~100 instructions in every workgroup.)
    for (int i0 = tid; i0 < n; i0 += DSP_NT * 16) {
        if (i0 != tid) load(i0);
#pragma unroll
        for (int u = 0; u < 16; u++) {
            const int a = i0 + DSP_NT * u;
            if (a < n) {
                const int e = clamp_id(v[u], E);
                sid[a] = (uint8_t)e;
                if (multi) atomicAdd(&cnt[wave][e], a < c0 ? 0x10001 : 1);
            }
        }
    }
    const int seg = (c1 - c0 + DSP_SEG - 1) / DSP_SEG, s0 = min(c1, c0 + wave * seg), s1 = min(c1, s0 + seg);
    const uint64_t lower = (1ull << lane) - 1ull;
    __syncthreads();
    if (multi) {
        if (tid < E) {
            unsigned sum = 0;
            for (int w = 0; w < DSP_SEG; w++) {
                sum += (unsigned)cnt[w][tid];
                cnt[w][tid] = 0;
            }
            tot[tid] = (int)(sum & 0xFFFFu);
            pre[tid] = (int)(sum >> 16);
        }
        __syncthreads();
    }
    for (int a0 = s0; a0 < s1; a0 += 64) {
        const int a = a0 + lane;
        const bool valid = a < s1;
        const int e = valid ? sid[a] : 0;
        const uint64_t m = same_expert_mask(e, valid, nbits);
        if (valid && (m & lower) == 0) cnt[wave][e] += __popcll(m);
    }
    __syncthreads();
    // per expert: each segment's start within the chunk's share, the total and the tile count
    int c = 0, tcount = 0;
    if (tid < E) {
        int run = pre[tid];
        for (int w = 0; w < DSP_SEG; w++) {
            const int h = cnt[w][tid];
            cnt[w][tid] = run;
            run += h;
        }
        c = gridDim.x > 1 ? tot[tid] : run;
        tcount = (c + A - 1) / A;
    }
    // exclusive scans of c and tcount over the experts (E <= 256: threads 0-255)
    const int v1 = wave_incl_scan_i(c), v2 = wave_incl_scan_i(tcount);
    if (lane == 63) {
        wsum[0][wave] = v1;
        wsum[1][wave] = v2;
    }
    __syncthreads();
    int b1 = 0, b2 = 0;
    for (int w = 0; w < min(wave, nwe); w++) {  // the later waves' sums are zero
        b1 += wsum[0][w];
        b2 += wsum[1][w];
    }
    if (tid < E) {
        toff[tid] = b1 + v1 - c;
        tb[tid] = b2 + v2 - tcount;
    }
    if (tid == PHX_MAX_EXPERTS_DEV - 1) {  // the scans' totals: experts past E hold zeros
        toff[E] = b1 + v1;
        tb[E] = b2 + v2;
        if (blockIdx.x == 0) *ntiles = b2 + v2;
    }
    __syncthreads();
    if (blockIdx.x == 0) {
        for (int e = tid; e <= E; e += DSP_NT) offsets[e] = toff[e];
        // the tiles, longest first (a grid runs its workgroups in tile order, so the short ones fill the
        // end): every full tile in expert order, then the partial ones in four size classes from the
        // largest, each in expert order
        const int nfull = tid < E ? c / A : 0, rem = tid < E ? c - nfull * A : 0;
        const int cls = rem ? min(4, (4 * rem + A - 1) / A) : 0;  // 1..4, 0: no partial tile
        int v[5] = {nfull, cls == 1, cls == 2, cls == 3, cls == 4};
        int inc[5];
#pragma unroll
        for (int q = 0; q < 5; q++) {
            const int x = wave_incl_scan_i(v[q]);
            inc[q] = x;
            if (lane == 63) tsum[q][wave] = x;
        }
        __syncthreads();
        int tot5[5], pre5[5];
#pragma unroll
        for (int q = 0; q < 5; q++) {
            tot5[q] = 0;
            pre5[q] = 0;
            for (int w = 0; w < nwe; w++) {  // the later waves' sums are zero
                tot5[q] += tsum[q][w];
                if (w < wave) pre5[q] += tsum[q][w];
            }
        }
        if (tid < E) {
            const int fb = pre5[0] + inc[0] - v[0];  // this expert's first full tile
            for (int q = 0; q < nfull; q++) tiles[fb + q] = Tile{tid, toff[tid] + q * A, A};
            if (cls) {
                int pos = tot5[0];
                for (int b = 4; b > cls; b--) pos += tot5[b];
                pos += cls == 1 ? pre5[1] + inc[1] - 1 : cls == 2 ? pre5[2] + inc[2] - 1
                       : cls == 3 ? pre5[3] + inc[3] - 1 : pre5[4] + inc[4] - 1;
                tiles[pos] = Tile{tid, toff[tid] + nfull * A, rem};
            }
        }
    }
    // placement of the chunk in assignment order
    for (int a0 = s0; a0 < s1; a0 += 64) {
        const int a = a0 + lane;
        const bool valid = a < s1;
        const int e = valid ? sid[a] : 0;
        const uint64_t m = same_expert_mask(e, valid, nbits);
        const int base = valid ? toff[e] + cnt[wave][e] : 0;
        if (valid) perm[base + __popcll(m & lower)] = a;
        __builtin_amdgcn_wave_barrier();  // every lane has read cnt before the batch's leaders advance it
        if (valid && (m & lower) == 0) cnt[wave][e] += __popcll(m);
    }
}

void launch_dispatch(hipStream_t st, int n, int E, int A, const int* ids, int* offsets, int* perm, Tile* tiles,
                     int* ntiles)
{
    (void)hipFuncSetAttribute((const void*)k_dispatch, hipFuncAttributeMaxDynamicSharedMemorySize, n);
    launch(k_dispatch, dim3((unsigned)((n + DSP_CH - 1) / DSP_CH)), dim3(DSP_NT), (uint32_t)n, st, n, E, A, ids, offsets,
           perm, tiles, ntiles);
}

// ------------------------------------------------------------------------------ grouped row products
// One workgroup = one tile (expert e, up to A assignments of its list) x 4 row groups; lane = row.
// Each lane walks its row's blocks in order and keeps, per assignment, the float chain of the
// reference row dot: sum += (float)isum * (d_w * d_x) (src/CpuRefGemma.cs:27-36, src/CpuRef.cs:106-115).
// Weights are read once per tile for all its assignments; activations are wave-uniform.

struct GroupArgs {
    const uint8_t* payload;
    const uint8_t* scale;
    int64_t mat_pay, mat_sc, rg_pay;
    int rg, nb, rows;
    Act act;
    const Tile* tiles;
    const int* ntiles;
    const int* perm;
    int act_div;
    float* out0;
    float* out1;
    int split, out_stride;
    bool paired;
    const void* grid;  // IQ types: the expanded codebook (64-bit words for IQ2_XXS / IQ2_S, 32-bit for IQ3_S)
    Act req;                       // req.q set: the paired gate|up kernel also writes gelu(g) * u as Q8_0 rows
    const float* gelu_tab = nullptr;
};

// Output of lane `lane` of row group rgi for assignment row a: natural row order, or for a paired
// gate|up matrix lanes 0-31 = gate output 32 rgi + lane, lanes 32-63 = the matching up output.
__device__ __forceinline__ void store_row(const GroupArgs& g, int rgi, int lane, int64_t a, float v)
{
    if (g.paired) {
        const int j = rgi * 32 + (lane & 31);
        if (j < g.split) (lane < 32 ? g.out0 : g.out1)[a * g.out_stride + j] = v;
    } else {
        const int row = rgi * 64 + lane;
        if (row < g.rows) {
            if (row < g.split) g.out0[a * g.out_stride + row] = v;
            else g.out1[a * g.out_stride + row - g.split] = v;
        }
    }
}

// The down input block rgi of assignment a from a paired row group's results (lanes 0-31 gate rows
// 32 rgi + l, lanes 32-63 the matching up rows): e = gelu(g) * u (src/GemmaCpu.cs:415) as a Q8_0 block
// (src/CpuRef.cs:49-62), what k_requant writes for it.  Wave-level.
__device__ __forceinline__ void requant_block(const GroupArgs& g, int rgi, int64_t a, float S)
{
    const int lane = threadIdx.x & 63, jj = rgi * 32 + (lane & 31);
    const float uv = __shfl_down(S, 32, 64);
    const float ev = lane < 32 ? gelu_ref(S, g.gelu_tab) * uv : 0.0f;
    float dval;
    int sum;
    const int q = q8_0_half(ev, &dval, &sum);
    if (lane < 32) {
        g.req.q[a * g.req.qstride + jj] = (int8_t)q;
        if (lane == 0) {
            g.req.d[a * g.req.dstride + rgi] = dval;
            g.req.s[a * g.req.sstride + rgi] = sum;
        }
    }
}

// Q4_0 / Q8_0 rows of up to QG_SHORT blocks: each lane walks its row's blocks in order, loading each
// block's payload and scale as it goes (a short row's many workgroups, no LDS, run in one round at
// several per CU and hide each other's loads).
template <int TYPE, int A>
__global__ __launch_bounds__(256) void k_grouped_q(GroupArgs g)
{
    const int tile = blockIdx.x;
    if (tile >= *g.ntiles) return;
    const Tile tl = g.tiles[tile];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rgi = blockIdx.y * 4 + wave;
    if (rgi >= g.rg) return;
    constexpr int PAY = TYPE == PHX_Q4_0_DEV ? 16 : 32;
    const uint8_t* wp = g.payload + tl.e * g.mat_pay + rgi * g.rg_pay + lane * PAY;
    const uint16_t* ws = (const uint16_t*)(g.scale + tl.e * g.mat_sc) + (int64_t)rgi * g.nb * 64 + lane;
    int arow[A];
    float acc[A];
#pragma unroll
    for (int i = 0; i < A; i++) {
        arow[i] = i < tl.cnt ? g.perm[tl.start + i] / g.act_div : 0;
        acc[i] = 0.0f;
    }
    for (int b = 0; b < g.nb; b++) {
        const float dw = h2f(ws[(int64_t)b * 64]);
        uint32_t wv[PAY / 4];
        {
            const uint4* src = (const uint4*)(wp + (int64_t)b * 64 * PAY);
#pragma unroll
            for (int c = 0; c < PAY / 16; c++) {
                uint4 t4 = src[c];
                wv[4 * c] = t4.x; wv[4 * c + 1] = t4.y; wv[4 * c + 2] = t4.z; wv[4 * c + 3] = t4.w;
            }
        }
#pragma unroll
        for (int i = 0; i < A; i++) {
            if (i < tl.cnt) {
                const int64_t r = arow[i];
                const uint32_t* xq = (const uint32_t*)(g.act.q + r * g.act.qstride + b * 32);
                int isum = 0;
                if (TYPE == PHX_Q4_0_DEV) {
#pragma unroll
                    for (int w = 0; w < 4; w++) {
                        isum = __builtin_amdgcn_sdot4((int)(wv[w] & 0x0F0F0F0Fu), (int)xq[w], isum, false);
                        isum = __builtin_amdgcn_sdot4((int)((wv[w] >> 4) & 0x0F0F0F0Fu), (int)xq[4 + w], isum, false);
                    }
                    isum -= 8 * g.act.s[r * g.act.sstride + b];
                } else {
#pragma unroll
                    for (int w = 0; w < 8; w++) isum = __builtin_amdgcn_sdot4((int)wv[w], (int)xq[w], isum, false);
                }
                const float dd = dw * g.act.d[r * g.act.dstride + b];
                acc[i] += (float)isum * dd;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < A; i++)
        if (i < tl.cnt) store_row(g, rgi, lane, g.perm[tl.start + i], acc[i]);
}

// Q4_0 / Q8_0 rows of more than QG_SHORT blocks.  The tile's activation rows (integers, scales and, for
// Q4_0, block sums) are staged in LDS, QG_CHB blocks at a time, and read back as wave-wide broadcasts.
// Each wave streams its row group's blocks (payload and scales) into a ring of QG_R slots of its own by
// direct global -> LDS loads, QG_R - 1 blocks ahead, and waits for a block by its own count of
// outstanding loads: no barrier, as no wave reads another's ring.  Every LDS read is explicit (a read the compiler emitted would first wait
// for all outstanding direct loads).  The launch gives each workgroup at least QG_LDS_MIN bytes of LDS:
// three workgroups per CU, which ran a layer's gate|up tiles (C5: ~720 workgroups) in one even round,
// 88 µs against 101 at four per CU and 106 for the row walk above.
constexpr int QG_R = 3, QG_CHB = 128;
template <int TYPE, int A>
__global__ __launch_bounds__(256) void k_grouped_q_ring(GroupArgs g)
{
    const int tile = blockIdx.x;
    if (tile >= *g.ntiles) return;  // uniform over the workgroup
    const Tile tl = g.tiles[tile];
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int rgi = blockIdx.y * 4 + wave;
    const bool live = rgi < g.rg;  // a wave past the last row group streams a clamped one, stores nothing
    constexpr int PAY = TYPE == PHX_Q4_0_DEV ? 16 : 32, NC = PAY / 16, NL = NC + 1;  // direct loads per block
    constexpr bool Q4 = TYPE == PHX_Q4_0_DEV;
    constexpr int SLOT = 64 * PAY + 256;  // a block's payload [64 rows][PAY], then its scales (4 B per lane)
    // LDS (sized by the launch for CH = min(nb, QG_CHB) blocks): the waves' rings [4][QG_R][SLOT], then the
    // activation chunk: integers [A][CH][32 B], scales [A][CH] and (Q4_0) block sums [A][CH]
    extern __shared__ __align__(16) unsigned char qg_lds[];
    const int nb = g.nb, rgc = min(rgi, g.rg - 1), CH = min(nb, QG_CHB);
    unsigned char* ringb = qg_lds;
    uint32_t* sq = (uint32_t*)(qg_lds + 4 * QG_R * SLOT);
    float* sd = (float*)(sq + A * CH * 8);
    int* ss = (int*)(sd + A * CH);
    const __amdgpu_buffer_rsrc_t r_w = buf_rsrc(g.payload + tl.e * g.mat_pay + rgc * g.rg_pay);
    const __amdgpu_buffer_rsrc_t r_s = buf_rsrc(g.scale + tl.e * g.mat_sc + (int64_t)rgc * nb * 64 * 2);
    const int cnt = min(tl.cnt, A);
    int arow[A];
    float acc[A];
#pragma unroll
    for (int i = 0; i < A; i++) {
        arow[i] = g.perm[tl.start + min(i, cnt - 1)] / g.act_div;
        acc[i] = 0.0f;
    }
    unsigned char* myring = ringb + wave * (QG_R * SLOT);
    auto issue = [&](int slot, int b) {  // block b (clamped: past the end a harmless reload)
        const uint32_t bc = (uint32_t)min(b, nb - 1);
        unsigned char* sl = myring + slot * SLOT;
#pragma unroll
        for (int c = 0; c < NC; c++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r_w, (lds_void_t)(sl + 1024 * c), 16, 16 * lane, bc * 64 * PAY + 1024 * c,
                                                     0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r_s, (lds_void_t)(sl + 64 * PAY), 2, 2 * lane, bc * 128, 0, 0);
    };
    const uint32_t a_w = (uint32_t)(uintptr_t)(lds_void_t)myring + PAY * lane;
    const uint32_t a_s = (uint32_t)(uintptr_t)(lds_void_t)myring + 64 * PAY + 4 * lane;
    const uint32_t a_q = (uint32_t)(uintptr_t)(lds_void_t)sq, a_d = (uint32_t)(uintptr_t)(lds_void_t)sd;
    const uint32_t a_ss = (uint32_t)(uintptr_t)(lds_void_t)ss;
    for (int c0 = 0; c0 < nb; c0 += QG_CHB) {
        // a chunk of activations into LDS (the loads' wait also lands the previous chunk's trailing ring
        // loads, so the ring restarts with nothing outstanding)
        const int nbc = min(QG_CHB, nb - c0);
        __syncthreads();  // the previous chunk's reads are done
        // the first chunk's first ring blocks go out before its activation loads (nothing is outstanding
        // yet), so the two cold reads overlap
        if (c0 == 0) {
#pragma unroll
            for (int r = 0; r < QG_R - 1; r++) issue(r, r);
        }
        // the tile's rows of the chunk (rows past cnt are never read): every load, then the stores
        constexpr int NQ = (A * QG_CHB * 2 + 255) / 256, ND = (A * QG_CHB + 255) / 256;
        uint4 qv[NQ];
        float dv[ND];
        int sv[ND];
#pragma unroll
        for (int u = 0; u < NQ; u++) {
            const int x = tid + 256 * u, i = x / (nbc * 2), y = x - i * nbc * 2;
            qv[u] = i < cnt ? ((const uint4*)(g.act.q + (int64_t)arow[i] * g.act.qstride + (int64_t)c0 * 32))[y]
                            : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int u = 0; u < ND; u++) {
            const int x = tid + 256 * u, i = x / nbc, y = x - i * nbc;
            dv[u] = i < cnt ? g.act.d[(int64_t)arow[i] * g.act.dstride + c0 + y] : 0.0f;
            sv[u] = Q4 && i < cnt ? g.act.s[(int64_t)arow[i] * g.act.sstride + c0 + y] : 0;
        }
#pragma unroll
        for (int u = 0; u < NQ; u++) {
            const int x = tid + 256 * u, i = x / (nbc * 2), y = x - i * nbc * 2;
            if (i < cnt) ((uint4*)(sq + i * CH * 8))[y] = qv[u];
        }
#pragma unroll
        for (int u = 0; u < ND; u++) {
            const int x = tid + 256 * u, i = x / nbc, y = x - i * nbc;
            if (i < cnt) {
                sd[i * CH + y] = dv[u];
                if (Q4) ss[i * CH + y] = sv[u];
            }
        }
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (c0 != 0) {
#pragma unroll
            for (int r = 0; r < QG_R - 1; r++) issue(r, c0 + r);
        }
        for (int bl = 0; bl < nbc; bl++) {
            const int b = c0 + bl, slot = bl % QG_R;
            // block b has landed once at most the QG_R - 2 later blocks' loads are outstanding; then the
            // slot read in the previous step (its reads waited for) takes block b + QG_R - 1
            __builtin_amdgcn_s_waitcnt((NL * (QG_R - 2)) | (0x7 << 4) | (0xF << 8));
            issue((bl + QG_R - 1) % QG_R, b + QG_R - 1);
            const uint32_t so = (uint32_t)(slot * SLOT);
            u32x4 w0 = ds_r128<0>(a_w + so), w1 = {0u, 0u, 0u, 0u};
            if constexpr (NC == 2) w1 = ds_r128<16>(a_w + so);
            uint32_t sv = ds_ru16<0>(a_s + so);
            u32x4 X0[A], X1[A];
            uint32_t XD[A], XS[A];
#pragma unroll
            for (int i = 0; i < A; i++) {
                X0[i] = ds_r128<0>(a_q + i * (CH * 32) + 32 * bl);
                X1[i] = ds_r128<16>(a_q + i * (CH * 32) + 32 * bl);
                XD[i] = ds_r32<0>(a_d + i * (CH * 4) + 4 * bl);
                XS[i] = Q4 ? ds_r32<0>(a_ss + i * (CH * 4) + 4 * bl) : 0u;
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            tie(w0);
            tie(w1);
            tie(sv);
#pragma unroll
            for (int i = 0; i < A; i++) {
                tie(X0[i]);
                tie(X1[i]);
                tie(XD[i]);
                tie(XS[i]);
            }
            const float dw = h2f(sv);
            const uint32_t w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
            for (int i = 0; i < A; i++) {
                if (i < cnt) {  // uniform
                    const uint32_t xq[8] = {X0[i].x, X0[i].y, X0[i].z, X0[i].w, X1[i].x, X1[i].y, X1[i].z, X1[i].w};
                    int isum = 0;
                    if constexpr (Q4) {
#pragma unroll
                        for (int k = 0; k < 4; k++) {
                            isum = __builtin_amdgcn_sdot4((int)(w[k] & 0x0F0F0F0Fu), (int)xq[k], isum, false);
                            isum = __builtin_amdgcn_sdot4((int)((w[k] >> 4) & 0x0F0F0F0Fu), (int)xq[4 + k], isum, false);
                        }
                        isum -= 8 * (int)XS[i];
                    } else {
#pragma unroll
                        for (int k = 0; k < 8; k++) isum = __builtin_amdgcn_sdot4((int)w[k], (int)xq[k], isum, false);
                    }
                    const float dd = dw * __uint_as_float(XD[i]);
                    acc[i] += (float)isum * dd;
                }
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0);  // the trailing ring loads land in this workgroup's LDS before it ends
    if (!live) return;  // wave-uniform
#pragma unroll
    for (int i = 0; i < A; i++)
        if (i < cnt) {  // uniform
            const int64_t a = g.perm[tl.start + i];
            store_row(g, rgi, lane, a, acc[i]);
            if (g.req.q) requant_block(g, rgi, a, acc[i]);
        }
}

// K-quant rows: DotK (src/CpuRefKQuants.cs:177-212) per (row, assignment): per super-block the eight
// integer lanes aux32[l] (element e contributes to lane e % 8), float lanes
// sums[l] += (d * yd) * aux32[l], the Q4_K / Q5_K min term sumf -= (dmin * yd) * sumi, finally sumf += sums[l].
template <int TYPE, int A>
__global__ __launch_bounds__(256) void k_grouped_k(GroupArgs g)
{
    const int tile = blockIdx.x;
    if (tile >= *g.ntiles) return;
    const Tile tl = g.tiles[tile];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rgi = blockIdx.y * 4 + wave;
    if (rgi >= g.rg) return;
    constexpr bool Q4K = TYPE == PHX_Q4_K_DEV, Q5K = TYPE == PHX_Q5_K_DEV;
    constexpr bool AFF = Q4K || Q5K;  // scales and mins per 32 (the min term); else 16 signed scales per 16
    constexpr int PAY = Q4K ? 144 : Q5K ? 176 : 208;
    const uint8_t* wp = g.payload + tl.e * g.mat_pay + rgi * g.rg_pay + lane * PAY;
    const uint8_t* wsb = g.scale + tl.e * g.mat_sc + ((int64_t)rgi * g.nb * 64 + lane) * (AFF ? 4 : 2);
    int arow[A];
    float sums[A][8], sumf[A];
#pragma unroll
    for (int i = 0; i < A; i++) {
        arow[i] = i < tl.cnt ? g.perm[tl.start + i] / g.act_div : 0;
        sumf[i] = 0.0f;
#pragma unroll
        for (int l = 0; l < 8; l++) sums[i][l] = 0.0f;
    }
    for (int b = 0; b < g.nb; b++) {
        uint32_t wv[PAY / 4];
        {
            const uint4* src = (const uint4*)(wp + (int64_t)b * 64 * PAY);
#pragma unroll
            for (int c = 0; c < PAY / 16; c++) {
                uint4 t4 = src[c];
                wv[4 * c] = t4.x; wv[4 * c + 1] = t4.y; wv[4 * c + 2] = t4.z; wv[4 * c + 3] = t4.w;
            }
        }
        float d, dmin = 0.0f;
        if (AFF) {
            uint32_t dm = *(const uint32_t*)(wsb + (int64_t)b * 64 * 4);
            d = h2f(dm & 0xFFFF);
            dmin = h2f(dm >> 16);
        } else {
            d = h2f(*(const uint16_t*)(wsb + (int64_t)b * 64 * 2));
        }
        // unpacked weight dwords
        uint32_t v[64];
        int sc[16], mn[8];
        if (AFF) {
#pragma unroll
            for (int w = 0; w < 32; w++) {
                v[2 * w] = wv[w] & 0x0F0F0F0Fu;
                v[2 * w + 1] = (wv[w] >> 4) & 0x0F0F0F0Fu;
            }
            if (Q5K)  // the fifth bits: bit l of byte mm of dword s belongs to value dword 8 s + l, byte mm
#pragma unroll
                for (int x = 0; x < 64; x++) v[x] |= ((wv[36 + x / 8] >> (x % 8)) & 0x01010101u) << 4;
#pragma unroll
            for (int s = 0; s < 8; s++) {
                sc[s] = (wv[32 + s / 4] >> (8 * (s % 4))) & 0xFF;
                mn[s] = (wv[34 + s / 4] >> (8 * (s % 4))) & 0xFF;
            }
        } else {
#pragma unroll
            for (int w = 0; w < 32; w++) {
                uint32_t lo0 = wv[w] & 0x0F0F0F0Fu, lo1 = (wv[w] >> 4) & 0x0F0F0F0Fu;
                int k0 = 2 * w, k1 = 2 * w + 1;
                uint32_t h0 = (wv[32 + k0 / 4] >> (2 * (k0 % 4))) & 0x03030303u;
                uint32_t h1 = (wv[32 + k1 / 4] >> (2 * (k1 % 4))) & 0x03030303u;
                v[k0] = lo0 | (h0 << 4);
                v[k1] = lo1 | (h1 << 4);
            }
#pragma unroll
            for (int s = 0; s < 16; s++) sc[s] = (int)(int8_t)((wv[48 + s / 4] >> (8 * (s % 4))) & 0xFF);
        }
#pragma unroll
        for (int i = 0; i < A; i++) {
            if (i < tl.cnt) {
                const int64_t r = arow[i];
                int aux[8];
#pragma unroll
                for (int l = 0; l < 8; l++) aux[l] = 0;
                if (AFF) {
                    const uint32_t* xq = (const uint32_t*)(g.act.q + r * g.act.qstride + b * 256);
#pragma unroll
                    for (int s = 0; s < 8; s++)
#pragma unroll
                        for (int l = 0; l < 8; l++)
                            aux[l] += sc[s] * __builtin_amdgcn_sdot4((int)v[s * 8 + l], (int)xq[s * 8 + l], 0, false);
                } else {
                    const uint32_t* xq = (const uint32_t*)(g.act.q + r * g.act.qstride + (int64_t)b * 512);
                    const int* cterm = g.act.s + r * g.act.sstride + b * 128;
#pragma unroll
                    for (int P = 0; P < 8; P++)
#pragma unroll
                        for (int l = 0; l < 8; l++) {
                            int pa = __builtin_amdgcn_sdot4((int)v[P * 8 + l], (int)xq[(P * 8 + l) * 2], cterm[(2 * P) * 8 + l], false);
                            int pb = __builtin_amdgcn_sdot4((int)v[P * 8 + l], (int)xq[(P * 8 + l) * 2 + 1],
                                                            cterm[(2 * P + 1) * 8 + l], false);
                            aux[l] += sc[2 * P] * pa;
                            aux[l] += sc[2 * P + 1] * pb;
                        }
                }
                const float yd = g.act.d[r * g.act.dstride + b];
                const float dd = d * yd;
#pragma unroll
                for (int l = 0; l < 8; l++) sums[i][l] += dd * (float)aux[l];
                if (AFF) {
                    const int* bs = g.act.s + r * g.act.sstride + b * 16;
                    int sumi = 0;
#pragma unroll
                    for (int j = 0; j < 16; j++) sumi += bs[j] * mn[j / 2];
                    const float dm = dmin * yd;
                    sumf[i] -= dm * (float)sumi;
                }
            }
        }
    }
#pragma unroll
    for (int i = 0; i < A; i++) {
        if (i < tl.cnt) {
            float s = sumf[i];
#pragma unroll
            for (int l = 0; l < 8; l++) s += sums[i][l];
            store_row(g, rgi, lane, g.perm[tl.start + i], s);
        }
    }
}

// Signs applied to four codebook bytes: bit j of nib set negates byte j.  The bit spread gives 0x01 in
// the negated bytes, times 0xFF the byte masks; (w ^ m) + (m & 0x01010101) negates those bytes without a
// carry between them, as every codebook byte is at least 1.
__device__ __forceinline__ uint32_t iq_signed(uint32_t w, uint32_t nib)
{
    const uint32_t m = ((nib * 0x00204081u) & 0x01010101u) * 0xFFu;
    return (w ^ m) + (m & 0x01010101u);
}

// ksigns of the IQ2_XXS format: seven stored sign bits and the eighth making the count even
__device__ __forceinline__ uint32_t iq_ksigns(uint32_t i) { return i | ((__builtin_popcount(i) & 1u) << 7); }

// IQ rows: DotIQ2XXS / DotIQ2S / DotIQ3S (src/CpuRefIQuants.cs:45-146) per (row, assignment).  Per
// super-block: the codebook points with their signs applied become 64 signed-byte dwords in element order
// (once per row), every assignment's integer sum bsum adds the 32-element (IQ2_S: 16-element) dot
// products times their odd scales, and sumf += (d * yd) * (float)bsum in super-block order; the IQ2 types
// return 0.125 * sumf.  The codebook sits in LDS (lanes look up different entries).
template <int TYPE, int A>
__global__ __launch_bounds__(256) void k_grouped_iq(GroupArgs g)
{
    constexpr bool IQ3 = TYPE == PHX_IQ3_S_DEV, IQ2S = TYPE == PHX_IQ2_S_DEV;
    constexpr int PAY = TYPE == PHX_IQ2_XXS_DEV ? 64 : IQ2S ? 80 : 112;
    constexpr int NW = TYPE == PHX_IQ2_XXS_DEV ? 512 : IQ2S ? 2048 : 512;  // codebook dwords
    __shared__ uint32_t cb[NW];
    for (int i = threadIdx.x; i < NW; i += 256) cb[i] = ((const uint32_t*)g.grid)[i];
    __syncthreads();
    const int tile = blockIdx.x;
    if (tile >= *g.ntiles) return;
    const Tile tl = g.tiles[tile];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rgi = blockIdx.y * 4 + wave;
    if (rgi >= g.rg) return;
    const uint8_t* wp = g.payload + tl.e * g.mat_pay + rgi * g.rg_pay + lane * PAY;
    const uint8_t* wsb = g.scale + tl.e * g.mat_sc + ((int64_t)rgi * g.nb * 64 + lane) * 2;
    int arow[A];
    float sumf[A];
#pragma unroll
    for (int i = 0; i < A; i++) {
        arow[i] = i < tl.cnt ? g.perm[tl.start + i] / g.act_div : 0;
        sumf[i] = 0.0f;
    }
    for (int b = 0; b < g.nb; b++) {
        uint32_t wv[PAY / 4];
        {
            const uint4* src = (const uint4*)(wp + (int64_t)b * 64 * PAY);
#pragma unroll
            for (int c = 0; c < PAY / 16; c++) {
                const uint4 t4 = src[c];
                wv[4 * c] = t4.x;
                wv[4 * c + 1] = t4.y;
                wv[4 * c + 2] = t4.z;
                wv[4 * c + 3] = t4.w;
            }
        }
        const float d = h2f(*(const uint16_t*)(wsb + (int64_t)b * 64 * 2));
        auto byte_at = [&](int o) -> uint32_t { return (wv[o >> 2] >> (8 * (o & 3))) & 0xFFu; };
        uint32_t v[64];
        int sc[16];  // scale per 16 elements
#pragma unroll
        for (int ib = 0; ib < 8; ib++) {
            if (TYPE == PHX_IQ2_XXS_DEV) {
                const uint32_t a0 = wv[2 * ib], a1 = wv[2 * ib + 1];
                sc[2 * ib] = sc[2 * ib + 1] = (int)(2 * (a1 >> 28) + 1);
#pragma unroll
                for (int l = 0; l < 4; l++) {
                    const uint32_t gi = (a0 >> (8 * l)) & 0xFFu, sg = iq_ksigns((a1 >> (7 * l)) & 127u);
                    v[8 * ib + 2 * l] = iq_signed(cb[2 * gi], sg & 15u);
                    v[8 * ib + 2 * l + 1] = iq_signed(cb[2 * gi + 1], sg >> 4);
                }
            } else if (IQ2S) {
                const uint32_t qh = byte_at(64 + ib), s8 = byte_at(72 + ib);
                sc[2 * ib] = 1 + 2 * (int)(s8 & 0xFu);
                sc[2 * ib + 1] = 1 + 2 * (int)(s8 >> 4);
#pragma unroll
                for (int l = 0; l < 4; l++) {
                    const uint32_t gi = byte_at(4 * ib + l) | ((qh << (8 - 2 * l)) & 0x300u);
                    const uint32_t sg = byte_at(32 + 4 * ib + l);
                    v[8 * ib + 2 * l] = iq_signed(cb[2 * gi], sg & 15u);
                    v[8 * ib + 2 * l + 1] = iq_signed(cb[2 * gi + 1], sg >> 4);
                }
            } else {
                const uint32_t h = byte_at(64 + ib), s8 = byte_at(104 + ib / 2);
                sc[2 * ib] = sc[2 * ib + 1] = 2 * (int)((ib & 1) ? s8 >> 4 : s8 & 0xFu) + 1;
#pragma unroll
                for (int l = 0; l < 4; l++) {
                    const uint32_t g1 = cb[byte_at(8 * ib + 2 * l) | ((h << (8 - 2 * l)) & 256u)];
                    const uint32_t g2 = cb[byte_at(8 * ib + 2 * l + 1) | ((h << (7 - 2 * l)) & 256u)];
                    const uint32_t sg = byte_at(72 + 4 * ib + l);
                    v[8 * ib + 2 * l] = iq_signed(g1, sg & 15u);
                    v[8 * ib + 2 * l + 1] = iq_signed(g2, sg >> 4);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < A; i++) {
            if (i < tl.cnt) {
                const int64_t r = arow[i];
                const uint32_t* xq = (const uint32_t*)(g.act.q + r * g.act.qstride + (int64_t)b * 256);
                int bsum = 0;
#pragma unroll
                for (int h16 = 0; h16 < 16; h16++) {
                    int s16 = 0;
#pragma unroll
                    for (int k = 0; k < 4; k++) s16 = __builtin_amdgcn_sdot4((int)v[4 * h16 + k], (int)xq[4 * h16 + k], s16, false);
                    bsum += sc[h16] * s16;
                }
                const float dd = d * g.act.d[r * g.act.dstride + b];
                sumf[i] += dd * (float)bsum;
            }
        }
    }
#pragma unroll
    for (int i = 0; i < A; i++)
        if (i < tl.cnt) store_row(g, rgi, lane, g.perm[tl.start + i], IQ3 ? sumf[i] : 0.125f * sumf[i]);
}

// dynamic LDS of k_grouped_q_ring<type, 4>: the rings and one activation chunk, at least QG_LDS_MIN
constexpr int QG_SHORT = 32, QG_LDS_MIN = 163840 / 4 + 1024;
static uint32_t grouped_q_lds(int type, int nb)
{
    const int pay = type == PHX_Q4_0_DEV ? 16 : 32, ch = std::min(nb, QG_CHB);
    const int need = 4 * QG_R * (64 * pay + 256) + 4 * ch * (32 + 4 + (type == PHX_Q4_0_DEV ? 4 : 0));
    return (uint32_t)std::max(need, QG_LDS_MIN);
}

void launch_grouped(hipStream_t st, const QMat& w, Act act, const Tile* tiles, const int* ntiles, int max_tiles, int A,
                    const int* perm, int act_div, float* out0, float* out1, int split, int out_stride,
                    const Act* req, const float* gelu_tab, int req_rows)
{
    GroupArgs g;
    g.payload = w.payload;
    g.scale = w.scale;
    g.mat_pay = w.mat_pay_stride();
    g.rg_pay = w.rg_pay;
    g.mat_sc = w.mat_sc_stride();
    g.rg = w.rg;
    g.nb = w.nb;
    g.rows = w.rows;
    g.act = act;
    g.tiles = tiles;
    g.ntiles = ntiles;
    g.perm = perm;
    g.act_div = act_div;
    g.out0 = out0;
    g.out1 = out1;
    g.split = split;
    g.out_stride = out_stride;
    g.paired = w.paired;
    g.grid = w.grid;
    // the down input in the ring kernel's epilogue where it covers every block of the row (paired Q4_0 /
    // Q8_0 rows past QG_SHORT blocks into Q8_0 rows with no padding blocks); else k_requant after it
    const bool fuse = req && w.paired && w.nb > QG_SHORT && (w.type == PHX_Q4_0_DEV || w.type == PHX_Q8_0_DEV) &&
                      req->fmt == ACT_Q8_0 && req->cols == 32 * w.rg && split == 32 * w.rg && !req->qh;
    if (fuse) {
        g.req = *req;
        g.gelu_tab = gelu_tab;
    }
    dim3 grid(max_tiles, (w.rg + 3) / 4);
    (void)A;  // the tile size the dispatch used: 4, the one instantiation
    switch (w.type) {
    case PHX_Q4_0_DEV:
        if (w.nb > QG_SHORT) launch((k_grouped_q_ring<PHX_Q4_0_DEV, 4>), grid, dim3(256), grouped_q_lds(w.type, w.nb), st, g);
        else launch((k_grouped_q<PHX_Q4_0_DEV, 4>), grid, dim3(256), 0, st, g);
        break;
    case PHX_Q8_0_DEV:
        if (w.nb > QG_SHORT) launch((k_grouped_q_ring<PHX_Q8_0_DEV, 4>), grid, dim3(256), grouped_q_lds(w.type, w.nb), st, g);
        else launch((k_grouped_q<PHX_Q8_0_DEV, 4>), grid, dim3(256), 0, st, g);
        break;
    case PHX_Q4_K_DEV: launch((k_grouped_k<PHX_Q4_K_DEV, 4>), grid, dim3(256), 0, st, g); break;
    case PHX_Q5_K_DEV: launch((k_grouped_k<PHX_Q5_K_DEV, 4>), grid, dim3(256), 0, st, g); break;
    case PHX_Q6_K_DEV: launch((k_grouped_k<PHX_Q6_K_DEV, 4>), grid, dim3(256), 0, st, g); break;
    case PHX_IQ2_XXS_DEV: launch((k_grouped_iq<PHX_IQ2_XXS_DEV, 4>), grid, dim3(256), 0, st, g); break;
    case PHX_IQ2_S_DEV: launch((k_grouped_iq<PHX_IQ2_S_DEV, 4>), grid, dim3(256), 0, st, g); break;
    case PHX_IQ3_S_DEV: launch((k_grouped_iq<PHX_IQ3_S_DEV, 4>), grid, dim3(256), 0, st, g); break;
    }
    if (req && !fuse) launch_requant(st, req_rows, split, out0, out1, gelu_tab, *req);
}

// ------------------------------------------------------------------------------ GELU-gated requant
// Per assignment row: e = gelu(g) * u (src/GemmaCpu.cs:415), zero padding up to act.cols, then the
// activation quantizer of the down weights (Q8_0 or Q8_K on entry to the down MatVec).
template <int NT>
__global__ __launch_bounds__(NT) void k_requant(int nf, const float* __restrict__ g, const float* __restrict__ u,
                                                const float* __restrict__ tab, Act act)
{
    extern __shared__ __align__(16) float sbuf[];
    const int64_t r = blockIdx.x;
    const int tid = threadIdx.x;
    // four values per thread and round (nf and cols are multiples of 32)
    const float4* g4 = (const float4*)(g + r * nf);
    const float4* u4 = (const float4*)(u + r * nf);
    for (int i4 = tid; i4 < act.cols / 4; i4 += NT) {
        float4 e = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (4 * i4 < nf) {
            const float4 gv = g4[i4], uv = u4[i4];
            e = make_float4(gelu_ref(gv.x, tab) * uv.x, gelu_ref(gv.y, tab) * uv.y, gelu_ref(gv.z, tab) * uv.z,
                            gelu_ref(gv.w, tab) * uv.w);
        }
        ((float4*)sbuf)[i4] = e;
    }
    __syncthreads();
    quantize_row<NT>(sbuf, act, r);
}

// Q8_K rows: one wave per super-block, all of a row's super-blocks at once up to 1024 threads (a row's
// values then need one load round); Q8_0 rows: 256 threads
void launch_requant(hipStream_t st, int rows, int nf, const float* g, const float* u, const float* tab, Act act)
{
    const size_t lds = (size_t)act.cols * sizeof(float);
    const int nsb = act.fmt == ACT_Q8_0 ? 0 : act.cols / 256;
    if (nsb >= 12) launch(k_requant<1024>, dim3(rows), dim3(1024), lds, st, nf, g, u, tab, act);
    else if (nsb >= 7) launch(k_requant<768>, dim3(rows), dim3(768), lds, st, nf, g, u, tab, act);
    else if (nsb >= 5) launch(k_requant<384>, dim3(rows), dim3(384), lds, st, nf, g, u, tab, act);
    else launch(k_requant<256>, dim3(rows), dim3(256), lds, st, nf, g, u, tab, act);
}

// ------------------------------------------------------------------------------ standalone quantizers
// KernelsQuant.Q80 / Q8K as an op of their own (src/KernelsQuant.cs:57-172, recorded by GemmaGpu.Quant,
// src/GemmaGpu.cs:442-461): rows x n inputs, each row quantized like CpuRef.QuantizeQ8_0
// (src/CpuRef.cs:49-62) or CpuRef.QuantizeQ8_K (src/CpuRefKQuants.cs:53-86) applied to
//   QZ_PLAIN x;  QZ_SILU silu(x) * u (CpuRef.Silu, src/CpuRef.cs:225-228: the exponential in double);
//   QZ_RMS   CpuRef.RmsNorm(x, w) (src/CpuRef.cs:183-191: (x * scale) * w, the row's certified mean);
//   QZ_GELU  gelu(x) * u (src/CpuRefGemma.cs:85-92).
// Outputs in CpuRef.Q8Activations' planar layout (src/CpuRef.cs:34-46): qs int8 [n] per row; Q8_0 d as
// fp16 bits [n/32]; Q8_K d float [n/256] and bsums int16 [n/16].  A workgroup takes ch elements of
// one row: QZ_CH, or in QZ_RMS the whole row up to 8192 (every workgroup forms its row's mean).
enum QzMode { QZ_PLAIN = 0, QZ_SILU = 1, QZ_RMS = 2, QZ_GELU = 3 };
constexpr int QZ_NT = 256, QZ_CH = 2048;

template <int MODE>
__device__ __forceinline__ float qz_in(float v, float a, float scale, const float* __restrict__ tab)
{
    if (MODE == QZ_SILU) return v / (1.0f + (float)exp(-(double)v)) * a;
    if (MODE == QZ_RMS) return v * scale * a;
    if (MODE == QZ_GELU) return gelu_ref(v, tab) * a;
    return v;
}

template <int MODE, bool K>
__global__ __launch_bounds__(QZ_NT) void k_quant(int n, int ch, float eps, const float* __restrict__ x,
                                                 const float* __restrict__ aux, const float* __restrict__ tab,
                                                 int8_t* __restrict__ qs, uint16_t* __restrict__ d16,
                                                 float* __restrict__ dk, int16_t* __restrict__ bsums, int* flags)
{
    const int64_t row = blockIdx.y;
    const int tid = threadIdx.x, c0 = blockIdx.x * ch, c1 = min(n, c0 + ch);
    const float* xr = x + row * n;
    const float* ar = MODE == QZ_RMS ? aux : aux + row * n;  // the norm weight is shared by the rows
    float scale = 0.0f;
    if (MODE == QZ_RMS) {
        __shared__ double red[QZ_NT / 64 + 1];
        scale = rms_scale_from_mean(mean_sq_cert<QZ_NT>(xr, n, red, flags), eps);
    }
    auto in4 = [&](int i) {
        const float4 v = *(const float4*)(xr + i);
        float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (MODE != QZ_PLAIN) a = *(const float4*)(ar + i);
        return make_float4(qz_in<MODE>(v.x, a.x, scale, tab), qz_in<MODE>(v.y, a.y, scale, tab),
                           qz_in<MODE>(v.z, a.z, scale, tab), qz_in<MODE>(v.w, a.w, scale, tab));
    };
    if (!K) {
        // eight lanes per 32-block, four values each; whole 8-lane groups run every round (shuffles)
        const int g = tid >> 3, l8 = tid & 7;
        for (int b0 = c0 / 32; b0 < c1 / 32; b0 += QZ_NT / 8) {
            const int b = b0 + g, bc = min(b, c1 / 32 - 1);
            float dval;
            int sum;
            const int qw = q8_0_oct(in4(bc * 32 + 4 * l8), &dval, &sum);
            if (b < c1 / 32) {
                *(int*)(qs + row * n + bc * 32 + 4 * l8) = qw;
                if (l8 == 0) d16[row * (n / 32) + bc] = (uint16_t)f2h_bits(dval);
            }
        }
        return;
    }
    // Q8_K: one wave per 256-block, lane l holds elements 4l..4l+3
    const int lane = tid & 63, wave = tid >> 6;
    for (int b = c0 / 256 + wave; b < c1 / 256; b += QZ_NT / 64) {
        const float4 v4 = in4(b * 256 + 4 * lane);
        const float v[4] = {v4.x, v4.y, v4.z, v4.w};
        // the reference's scan: the first element of largest |x| (strict '>', from 0)
        float amax = 0.0f, vmax = 0.0f;
        int imax = 1 << 30;
#pragma unroll
        for (int j = 0; j < 4; j++)
            if (fabsf(v[j]) > amax) {
                amax = fabsf(v[j]);
                vmax = v[j];
                imax = 4 * lane + j;
            }
        // the wave's first largest |x| by DPP steps (lanes outside a step's rows keep their own triple),
        // lane 63 ending with the result
        auto step = [&](auto C, auto RM) {
            constexpr int CTRL = decltype(C)::value, ROWMASK = decltype(RM)::value;
            const float oa = dpp_f<CTRL, ROWMASK>(amax, amax), ov = dpp_f<CTRL, ROWMASK>(vmax, vmax);
            const int oi = dpp_i<CTRL, ROWMASK>(imax, imax);
            if (oa > amax || (oa == amax && oi < imax)) {
                amax = oa;
                vmax = ov;
                imax = oi;
            }
        };
        step(ic<0xb1>{}, ic<0xf>{});
        step(ic<0x4e>{}, ic<0xf>{});
        step(ic<0x141>{}, ic<0xf>{});
        step(ic<0x140>{}, ic<0xf>{});
        step(ic<0x142>{}, ic<0xa>{});
        step(ic<0x143>{}, ic<0xc>{});
        amax = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(amax), 63));
        vmax = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(vmax), 63));
        const float iscale = amax == 0.0f ? 0.0f : -127.0f / vmax;
        int q[4], sm = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            q[j] = amax == 0.0f ? 0 : min(nearest_int(iscale * v[j]), 127);
            sm += q[j];
        }
        *(int*)(qs + row * n + b * 256 + 4 * lane) =
            (q[0] & 0xFF) | ((q[1] & 0xFF) << 8) | ((q[2] & 0xFF) << 16) | (int)((unsigned)q[3] << 24);
        sm += dpp_i<0xb1>(sm, sm);  // 4-lane sum: quad swaps
        sm += dpp_i<0x4e>(sm, sm);
        if (bsums && (lane & 3) == 0) bsums[row * (n / 16) + b * 16 + (lane >> 2)] = (int16_t)sm;
        if (lane == 0) dk[row * (n / 256) + b] = amax == 0.0f ? 0.0f : 1.0f / iscale;
    }
}

int launch_quant(hipStream_t st, int fmt_k, int mode, int rows, int n, float eps, const float* x, const float* aux,
                 const float* tab, int8_t* qs, uint16_t* d16, float* dk, int16_t* bsums, int* flags)
{
    // rows are independent outside QZ_RMS and the outputs are row-major: quantize them as one row
    if (mode != QZ_RMS && (int64_t)rows * n <= (int64_t)1 << 30) {
        n *= rows;
        rows = 1;
    }
    const int ch = mode == QZ_RMS && n <= 8192 ? n : QZ_CH;  // a multiple of 256 or of 32 as the format needs
    const dim3 grid((n + ch - 1) / ch, rows), blk(QZ_NT);
#define QZ_L(M, K) launch((k_quant<M, K>), grid, blk, 0, st, n, ch, eps, x, aux, tab, qs, d16, dk, bsums, flags)
    switch (mode * 2 + (fmt_k ? 1 : 0)) {
    case 0: QZ_L(QZ_PLAIN, false); break;
    case 1: QZ_L(QZ_PLAIN, true); break;
    case 2: QZ_L(QZ_SILU, false); break;
    case 3: QZ_L(QZ_SILU, true); break;
    case 4: QZ_L(QZ_RMS, false); break;
    case 5: QZ_L(QZ_RMS, true); break;
    case 6: QZ_L(QZ_GELU, false); break;
    case 7: QZ_L(QZ_GELU, true); break;
    default: return -1;
    }
#undef QZ_L
    return 0;
}

// ------------------------------------------------------------------------------ norm + residual (+ quant)
// KernelsGemma.NormAdd / NormAddQuant (src/KernelsGemma.cs:126-226) with the CPU path's rounding
// (GemmaCpu.PostAndFfn, src/GemmaCpu.cs:353-356 and 367; then the next RmsNorm and MatVec's Q8_0 input,
// src/CpuRef.cs:49-62, 183-191), one workgroup per row: x = x + rmsnorm(y, w) (the term rounded as
// CpuRef.RmsNorm forms it), times s when s != 1; with w2, the Q8_0 quantization of rmsnorm(x_new, w2)
// into qs / d16 (fp16 bits).  Both means of squares are certified (mean_sq_cert).
constexpr int NA_NT = 512;

__global__ __launch_bounds__(NA_NT) void k_norm_add(int n, float eps, float s, float* __restrict__ x,
                                                    const float* __restrict__ y, const float* __restrict__ w,
                                                    const float* __restrict__ w2, int8_t* __restrict__ qs,
                                                    uint16_t* __restrict__ d16, int* flags)
{
    extern __shared__ __align__(16) float sx[];  // the new x row
    __shared__ double red[NA_NT / 64 + 1];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x, n4 = n / 4;
    float* xr = x + row * n;
    const float* yr = y + row * n;
    const float sc1 = rms_scale_from_mean(mean_sq_cert<NA_NT>(yr, n, red, flags), eps);
    for (int i4 = tid; i4 < n4; i4 += NA_NT) {
        const float4 xv = ((const float4*)xr)[i4], yv = ((const float4*)yr)[i4], wv = ((const float4*)w)[i4];
        float4 v = make_float4(xv.x + yv.x * sc1 * wv.x, xv.y + yv.y * sc1 * wv.y, xv.z + yv.z * sc1 * wv.z,
                               xv.w + yv.w * sc1 * wv.w);
        if (s != 1.0f) v = make_float4(v.x * s, v.y * s, v.z * s, v.w * s);
        ((float4*)xr)[i4] = v;
        ((float4*)sx)[i4] = v;
    }
    if (!w2) return;  // uniform
    __syncthreads();
    const float sc2 = rms_scale_from_mean(mean_sq_cert<NA_NT>(sx, n, red, flags), eps);
    // eight lanes per 32-block; whole 8-lane groups run every round (shuffles)
    const int g = tid >> 3, l8 = tid & 7, nb = n / 32;
    for (int b0 = 0; b0 < nb; b0 += NA_NT / 8) {
        const int b = b0 + g, bc = min(b, nb - 1);
        const float4 xv = *(const float4*)(sx + bc * 32 + 4 * l8), wv = *(const float4*)(w2 + bc * 32 + 4 * l8);
        float dval;
        int sum;
        const int qw = q8_0_oct(make_float4(xv.x * sc2 * wv.x, xv.y * sc2 * wv.y, xv.z * sc2 * wv.z,
                                            xv.w * sc2 * wv.w),
                                &dval, &sum);
        if (b < nb) {
            *(int*)(qs + row * n + bc * 32 + 4 * l8) = qw;
            if (l8 == 0) d16[row * nb + bc] = (uint16_t)f2h_bits(dval);
        }
    }
}

void launch_norm_add(hipStream_t st, int rows, int n, float eps, float s, float* x, const float* y, const float* w,
                     const float* w2, int8_t* qs, uint16_t* d16, int* flags)
{
    launch(k_norm_add, dim3(rows), dim3(NA_NT), (size_t)n * sizeof(float), st, n, eps, s, x, y, w, w2, qs, d16, flags);
}

// ------------------------------------------------------------------------------ dense matvec
// KernelsGemma.MatVecQ4_0 / the Q8_0 matvec as GemmaGpu.MatVec records them (src/KernelsGemma.cs:244-306,
// src/GemmaGpu.cs:463-476), with CpuRef's rounding (MatVecQ4_0, src/CpuRefGemma.cs:12-40; MatVecQ8_0,
// src/CpuRef.cs:91-119): y[t][r] = the float sum, in block order from 0, of (float)isum_b * (d_w * d_x),
// isum_b the integer dot of weight block b of row r with input block b of token t (planar Q8_0 input as
// phx_quant_q8_0 writes it).  Rows as the GGUF file holds them (row r at r * row_bytes).  One wave per
// row: the row staged in LDS by coalesced 2-byte loads, one block per lane and round, the terms added in
// block order by lane 0.
constexpr int MV_NT = 256, MV_ROWS = MV_NT / 64;

template <int TYPE>  // PHX_Q4_0_DEV or PHX_Q8_0_DEV
__global__ __launch_bounds__(MV_NT) void k_matvec(int rows, int nb, const uint8_t* __restrict__ w,
                                                  const int8_t* __restrict__ xq, const uint16_t* __restrict__ xd,
                                                  float* __restrict__ y)
{
    constexpr int BB = TYPE == PHX_Q4_0_DEV ? 18 : 34;
    extern __shared__ __align__(16) uint8_t mv[];  // [MV_ROWS][terms nb floats], then [MV_ROWS][row bytes]
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, rb = nb * BB;
    const int r = blockIdx.x * MV_ROWS + wave;  // wave-uniform
    const int64_t t = blockIdx.y;
    float* terms = (float*)mv + wave * nb;
    uint16_t* srow = (uint16_t*)((float*)mv + MV_ROWS * nb) + wave * (rb / 2);
    // the lane's first activation block, loaded beside the row (it does not depend on the weights)
    const int4* qx0 = (const int4*)(xq + (t * nb + min(lane, nb - 1)) * 32);
    const int4 xa0 = qx0[0], xb0 = qx0[1];
    if (r < rows) {
        const uint16_t* src = (const uint16_t*)(w + (int64_t)r * rb);
        for (int i = lane; i < rb / 2; i += 64) srow[i] = src[i];
    }
    __syncthreads();
    if (r < rows) {
        for (int b = lane; b < nb; b += 64) {
            const uint16_t* blk = srow + b * (BB / 2);  // d, then the payload as 2-byte halves
            const int4* qx4 = (const int4*)(xq + (t * nb + b) * 32);
            const int4 xa = b == lane ? xa0 : qx4[0], xb = b == lane ? xb0 : qx4[1];
            const int x[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
            int isum = 0;
            if (TYPE == PHX_Q4_0_DEV) {
                // word k holds the nibbles of elements 4k..4k+3 (low) and 4k+16..4k+19 (high); each
                // nibble n becomes the signed byte n - 8 (bias through the top bit)
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const uint32_t q = (uint32_t)blk[1 + 2 * k] | ((uint32_t)blk[2 + 2 * k] << 16);
                    const int lo = (int)((((q & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u);
                    const int hi = (int)(((((q >> 4) & 0x0F0F0F0Fu) | 0x80808080u) - 0x08080808u) ^ 0x80808080u);
                    isum = __builtin_amdgcn_sdot4(lo, x[k], isum, false);
                    isum = __builtin_amdgcn_sdot4(hi, x[k + 4], isum, false);
                }
            } else {
#pragma unroll
                for (int k = 0; k < 8; k++)
                    isum = __builtin_amdgcn_sdot4((int)((uint32_t)blk[1 + 2 * k] | ((uint32_t)blk[2 + 2 * k] << 16)),
                                                  x[k], isum, false);
            }
            terms[b] = (float)isum * (h2f(blk[0]) * h2f(xd[t * nb + b]));
        }
    }
    __syncthreads();
    if (r < rows && lane == 0) {
        // sixteen terms read at a time (every read issued before the first add), added in order
        float sum = 0.0f;
        int b = 0;
        for (; b + 16 <= nb; b += 16) {
            float v[16];
#pragma unroll
            for (int j = 0; j < 16; j++) v[j] = terms[b + j];
#pragma unroll
            for (int j = 0; j < 16; j++) sum += v[j];
        }
        for (; b < nb; b++) sum += terms[b];
        y[t * rows + r] = sum;
    }
}

size_t matvec_lds(int type, int nb) { return (size_t)MV_ROWS * nb * (4 + (type == PHX_Q4_0_DEV ? 18 : 34)); }

void launch_matvec(hipStream_t st, int type, int rows, int nb, int T, const uint8_t* w, const int8_t* xq,
                   const uint16_t* xd, float* y)
{
    const dim3 grid((rows + MV_ROWS - 1) / MV_ROWS, T);
    if (type == PHX_Q4_0_DEV)
        launch(k_matvec<PHX_Q4_0_DEV>, grid, dim3(MV_NT), matvec_lds(type, nb), st, rows, nb, w, xq, xd, y);
    else
        launch(k_matvec<PHX_Q8_0_DEV>, grid, dim3(MV_NT), matvec_lds(type, nb), st, rows, nb, w, xq, xd, y);
}

// ------------------------------------------------------------------------------ combine, norms, residual
// Per token: acc = sum_j yd[t*k+j] * w_j in rank order (src/GemmaCpu.cs:418, each term rounded then
// added), out = rmsnorm(shared) * post1 + rmsnorm(acc) * post2 (src/GemmaCpu.cs:384,420-421), and
// optionally x += rmsnorm(out) * post_ffw_norm (src/GemmaCpu.cs:355-356).  For rows wider than the
// one-round combine's 4096 columns (kernels_decode.hip: launch_combine): 256 threads over the row.
__global__ __launch_bounds__(256) void k_combine_wide(int d, int k, float eps, const float* __restrict__ yd,
                                                 const float* __restrict__ w, const float* __restrict__ shared,
                                                 const float* __restrict__ post1, const float* __restrict__ post2,
                                                 float* __restrict__ out, float* __restrict__ xres,
                                                 const float* __restrict__ post_ffw, int* flags)
{
    extern __shared__ float sbuf[];  // [2][d]
    __shared__ double red[256];
    const int t = blockIdx.x, tid = threadIdx.x, d4 = d / 4;  // d % 32 == 0
    float* acc = sbuf;
    float* o = sbuf + d;
    const float4* y4 = (const float4*)yd + (int64_t)t * k * d4;
    const float* wt = w + (int64_t)t * k;
    // acc = sum_j w_j * yd_j in rank order (each term rounded, then added); four elements per thread,
    // the loads of eight ranks issued before their use
    for (int i4 = tid; i4 < d4; i4 += 256) {
        float4 a = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int j0 = 0; j0 < k; j0 += 8) {
            float4 yv[8];
            float wj[8];
#pragma unroll
            for (int jj = 0; jj < 8; jj++) {
                const int j = min(j0 + jj, k - 1);
                yv[jj] = y4[(int64_t)j * d4 + i4];
                wj[jj] = wt[j];
            }
#pragma unroll
            for (int jj = 0; jj < 8; jj++) {
                if (j0 + jj < k) {
                    a.x += yv[jj].x * wj[jj];
                    a.y += yv[jj].y * wj[jj];
                    a.z += yv[jj].z * wj[jj];
                    a.w += yv[jj].w * wj[jj];
                }
            }
        }
        ((float4*)acc)[i4] = a;
    }
    __syncthreads();
    const float s2 = rms_scale_from_mean(mean_sq_cert<256>(acc, d, red, flags), eps);
    float s1 = 0.0f;
    const float* sh = shared ? shared + (int64_t)t * d : nullptr;
    if (sh) s1 = rms_scale_from_mean(mean_sq_cert<256>(sh, d, red, flags), eps);
    for (int i = tid; i < d; i += 256) {
        float mlp = sh ? sh[i] * s1 * post1[i] : 0.0f;
        float v = mlp + acc[i] * s2 * post2[i];
        out[(int64_t)t * d + i] = v;
        o[i] = v;
    }
    if (xres) {
        __syncthreads();
        const float s3 = rms_scale_from_mean(mean_sq_cert<256>(o, d, red, flags), eps);
        for (int i = tid; i < d; i += 256) xres[(int64_t)t * d + i] += o[i] * s3 * post_ffw[i];
    }
}

void launch_combine_wide(hipStream_t st, int T, int d, int k, float eps, const float* yd, const float* w,
                         const float* shared, const float* post1, const float* post2, float* out, float* xres,
                         const float* post_ffw, int* flags)
{
    launch(k_combine_wide, dim3(T), dim3(256), (size_t)2 * d * sizeof(float), st, d, k, eps, yd, w, shared, post1,
           post2, out, xres, post_ffw, flags);
}

// ------------------------------------------------------------------------------ streaming read
// Reads `n16` 16-byte words with coalesced 128-bit loads and folds them into one word per thread
// (written only when it equals a sentinel, so the loads cannot be elided): the achievable HBM read
// rate of the box, the denominator check of the roofline.
__global__ __launch_bounds__(256) void k_stream_read(const uint4* __restrict__ src, int64_t n16, uint32_t* sink)
{
    uint32_t acc = 0;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
        uint4 v = src[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

void launch_stream_read(hipStream_t st, const void* src, int64_t bytes, uint32_t* sink)
{
    launch(k_stream_read, dim3(256 * 8), dim3(256), 0, st, (const uint4*)src, bytes / 16, sink);
}

// Streaming copy of n16 16-byte words: a kernel of known traffic (bytes read = bytes written) for
// scaling the memory counters of a profiler.
__global__ __launch_bounds__(256) void k_stream_copy(uint4* __restrict__ dst, const uint4* __restrict__ src, int64_t n16)
{
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

void launch_stream_copy(hipStream_t st, void* dst, const void* src, int64_t bytes)
{
    launch(k_stream_copy, dim3(256 * 8), dim3(256), 0, st, (uint4*)dst, (const uint4*)src, bytes / 16);
}

// Planar Q8_0 rows (qs int8 [rows][n] and fp16 scale bits [rows][n/32], the layout phx_quant_q8_0
// writes) into the grouped kernels' activation arrays: each block's scale as a float, the sum of its
// integers (the Q4_0 offset term of the VALU kernels) and, when a.qh is set, the integers as exact
// fp16 (the matrix-core operands).  An 8-lane group per block, four integers per lane.
__global__ __launch_bounds__(256) void k_planar_act(int64_t nblk, int nb, const int8_t* __restrict__ qs,
                                                    const uint16_t* __restrict__ d, Act a)
{
    const int64_t g = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 3;
    const int l8 = threadIdx.x & 7;
    const bool ok = g < nblk;
    const int64_t gc = ok ? g : nblk - 1;  // every lane takes part in the group's shuffles
    const uint32_t w = ((const uint32_t*)qs)[gc * 8 + l8];
    const int q0 = (int8_t)(w & 0xFF), q1 = (int8_t)((w >> 8) & 0xFF), q2 = (int8_t)((w >> 16) & 0xFF),
              q3 = (int8_t)(w >> 24);
    int sm = q0 + q1 + q2 + q3;
    sm += dpp_i<0xb1>(sm, sm);  // 8-lane sum: quad swaps, then the other quad (half-row mirror)
    sm += dpp_i<0x4e>(sm, sm);
    sm += dpp_i<0x141>(sm, sm);
    if (!ok) return;
    const int64_t t = g / nb;
    const int b = (int)(g - t * nb);
    if (l8 == 0) {
        a.d[t * a.dstride + b] = h2f(d[g]);
        a.s[t * a.sstride + b] = sm;
    }
    if (a.qh) {
        const uint32_t h01 = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)q0) |
                             ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)q1) << 16);
        const uint32_t h23 = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)q2) |
                             ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)q3) << 16);
        *(uint2*)(a.qh + t * a.qhstride + b * 32 + 4 * l8) = make_uint2(h01, h23);
    }
}

void launch_planar_act(hipStream_t st, int rows, int n, const int8_t* qs, const uint16_t* d, Act a)
{
    const int64_t nblk = (int64_t)rows * (n / 32);
    launch(k_planar_act, dim3((unsigned)((nblk * 8 + 255) / 256)), dim3(256), 0, st, nblk, n / 32, qs, d, a);
}

// Planar Q8_K rows (qs int8 [rows][n] in element order and the float scale [rows][n/256], the layout
// phx_quant_q8_k writes) into the K-quant kernels' activation arrays (ACT_K4 / ACT_K6 orders, the sums
// of 16, and with a.qh / a.bh set the matrix cores' fp16 copies).  One wave per 256-block.
__global__ __launch_bounds__(256) void k_planar_act_k(int64_t nblk, int nb, const int8_t* __restrict__ qs,
                                                      const float* __restrict__ d, Act a)
{
    __shared__ uint32_t qsm[4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t g = (int64_t)blockIdx.x * 4 + wave;
    if (g >= nblk) return;  // wave-uniform; the block store synchronises within the wave only
    const int64_t t = g / nb;
    const int b = (int)(g - t * nb);
    const uint32_t pk = ((const uint32_t*)qs)[g * 64 + lane];
    const float dval = d[g];
    if (lane == 0) a.d[t * a.dstride + b] = dval;
    store_q8k_block(a, t, b, lane, pk, qsm[wave], dval);
}

void launch_planar_act_k(hipStream_t st, int rows, int n, const int8_t* qs, const float* d, Act a)
{
    const int64_t nblk = (int64_t)rows * (n / 256);
    launch(k_planar_act_k, dim3((unsigned)((nblk + 3) / 4)), dim3(256), 0, st, nblk, n / 256, qs, d, a);
}

// Copy of a small buffer (bytes a multiple of 16) by a few workgroups: the host-buffer path's staging
// between pinned host rows and the device rows, as graph nodes rather than DMA copies.
__global__ __launch_bounds__(256) void k_copy16(uint4* __restrict__ dst, const uint4* __restrict__ src, int64_t n16)
{
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

void launch_copy_small(hipStream_t st, void* dst, const void* src, int64_t bytes)
{
    const int64_t n16 = bytes / 16;
    launch(k_copy16, dim3((unsigned)std::min<int64_t>(64, (n16 + 255) / 256)), dim3(256), 0, st, (uint4*)dst,
           (const uint4*)src, n16);
}

// The last copies of a host-buffer call, by one workgroup: out (and x with the residual) to the pinned
// rows, then the call's completion word: the next count (never zero, the word's initial value), stored
// after a system-scope fence so the host, which polls the word, reads whole rows once it changes.
__global__ __launch_bounds__(1024) void k_copy_done(uint4* __restrict__ d0, const uint4* __restrict__ s0,
                                                    uint4* __restrict__ d1, const uint4* __restrict__ s1, int64_t n16,
                                                    uint32_t* __restrict__ ctr, uint32_t* done)
{
    for (int64_t i = threadIdx.x; i < n16; i += 1024) d0[i] = s0[i];
    if (d1)
        for (int64_t i = threadIdx.x; i < n16; i += 1024) d1[i] = s1[i];
    __syncthreads();
    if (threadIdx.x == 0) {
        const uint32_t v = ctr[0] == 0xFFFFFFFFu ? 1u : ctr[0] + 1u;
        ctr[0] = v;
        __threadfence_system();
        __hip_atomic_store(done, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

void launch_copy_done(hipStream_t st, void* d0, const void* s0, void* d1, const void* s1, int64_t bytes, uint32_t* ctr,
                      uint32_t* done)
{
    launch(k_copy_done, dim3(1), dim3(1024), 0, st, (uint4*)d0, (const uint4*)s0, (uint4*)d1, (const uint4*)s1,
           bytes / 16, ctr, done);
}

// Fill n 32-bit words with v: clears workspace that must start at zero with a kernel rather than a
// memset node, so the enqueued work stays a plain kernel when a caller captures it into a graph.
__global__ __launch_bounds__(256) void k_fill_u32(uint32_t* __restrict__ p, int64_t n, uint32_t v)
{
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) p[i] = v;
}

void launch_fill_u32(hipStream_t st, uint32_t* p, int64_t n, uint32_t v)
{
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 1024);
    launch(k_fill_u32, dim3((unsigned)std::max<int64_t>(blocks, 1)), dim3(256), 0, st, p, n, v);
}

// ------------------------------------------------------------------------------ arithmetic self-test
typedef float st_f4 __attribute__((ext_vector_type(4)));
__global__ void k_selftest(int op, int n, const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ out,
                           const float* __restrict__ tab)
{
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (op >= 8) {  // one 16 x 16 x 4 fp32 matrix-core product per 64 elements (n a multiple of 64)
        if (i - (i & 63) >= n) return;  // whole waves
        const float c = op == 9 ? 1.0f : 0.0f;
        const st_f4 d = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[i], st_f4{c, c, c, c}, 0, 0, 0);
        out[i] = d[0];
        return;
    }
    if (i >= n) return;
    float x = a[i], y = b[i], r = 0.0f;
    switch (op) {
    case 0: r = x / y; break;
    case 1: r = rms_scale_from_mean(x, y); break;
    case 2: r = (float)((double)x / (double)y); break;
    case 3: r = roundf(x); break;
    case 4: r = (float)f2h_bits(x); break;
    case 5: r = (float)nearest_int(x); break;
    case 6: r = gelu_ref(x, tab); break;
    case 7: r = h2f((uint32_t)x); break;
    }
    out[i] = r;
}

void launch_selftest(hipStream_t st, int op, int n, const float* a, const float* b, float* out, const float* tab)
{
    launch(k_selftest, dim3((n + 255) / 256), dim3(256), 0, st, op, n, a, b, out, tab);
}

// one wave per row of m floats: the row's sequential double sum of squares (seq_sum_sq_wave), its two
// 32-bit halves in out[2 r] (low) and out[2 r + 1] (high)
__global__ __launch_bounds__(64) void k_selftest_seq(int m, const float* __restrict__ a, float* __restrict__ out)
{
    const int r = blockIdx.x;
    const double q = seq_sum_sq_wave(a + (int64_t)r * m, m);
    if (threadIdx.x == 0) {
        const unsigned long long u = (unsigned long long)__double_as_longlong(q);
        out[2 * r] = __uint_as_float((unsigned)u);
        out[2 * r + 1] = __uint_as_float((unsigned)(u >> 32));
    }
}

void launch_selftest_seq(hipStream_t st, int m, int rows, const float* a, float* out)
{
    launch(k_selftest_seq, dim3(rows), dim3(64), 0, st, m, a, out);
}

}  // namespace phx

#ifdef PHX_TIMELINE
// the instrumented build's clock-stamp table of this file's kernels (as phxdbg_timeline)
extern "C" __attribute__((visibility("default"))) int phxdbg_timeline_general(unsigned long long* host, size_t n, int clear)
{
    const size_t all = sizeof(phx::phx_tl) / sizeof(phx::phx_tl[0]);
    if (host && hipMemcpyFromSymbol(host, HIP_SYMBOL(phx::phx_tl), std::min(n, all) * 8, 0, hipMemcpyDeviceToHost) != hipSuccess)
        return -1;
    if (clear) {
        static unsigned long long* zero = nullptr;
        if (!zero) zero = (unsigned long long*)calloc(all, 8);
        if (hipMemcpyToSymbol(HIP_SYMBOL(phx::phx_tl), zero, all * 8, 0, hipMemcpyHostToDevice) != hipSuccess) return -1;
    }
    return (int)all;
}
#endif
