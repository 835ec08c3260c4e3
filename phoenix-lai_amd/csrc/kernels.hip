// gfx950 kernels of the MoE FFN layer.  wave64 throughout; built with -ffp-contract=off so every
// float expression keeps the reference CPU path's rounding sequence (src/GemmaCpu.cs:376-422 over
// src/CpuRef*.cs): products and sums that the reference evaluates in a fixed order are evaluated
// in that order (per-row block chains, the router's dot chain, the rank-ordered combine), and the
// double-precision sums of squares of RmsNorm are reproduced through a certified error bound with
// an exact sequential fallback.
#include "device_common.h"

namespace phx {

// ------------------------------------------------------------------------------ activation quantizers

// Quantize one row (in LDS, `cols` floats) into format act, row index `row`.  Block-level (NT threads).
//  Q8_0: CpuRef.QuantizeQ8_0 (src/CpuRef.cs:49-62), plus the block sum of q for the Q4_0 offset.
//  K4/K6: CpuRef.QuantizeQ8_K (src/CpuRefKQuants.cs:53-86), stored in the dot-product orders.
template <int NT>
__device__ void quantize_row(const float* v, Act act, int64_t row)
{
    const int tid = threadIdx.x;
    if (act.fmt == ACT_Q8_0) {
        int nb = act.cols / 32;
        for (int b = tid; b < nb; b += NT) {
            const float* x = v + b * 32;
            float amax = 0.0f;
            for (int j = 0; j < 32; j++) { float a = fabsf(x[j]); if (a > amax) amax = a; }
            float d = amax / 127.0f;
            float id = d != 0.0f ? 1.0f / d : 0.0f;
            uint32_t dh = f2h_bits(d);
            uint32_t w[8];
            int sum = 0;
            for (int j = 0; j < 32; j += 4) {
                uint32_t pk = 0;
                for (int m = 0; m < 4; m++) {
                    int q = (int)roundf(x[j + m] * id);
                    sum += q;
                    pk |= (uint32_t)(q & 0xFF) << (8 * m);
                }
                w[j / 4] = pk;
            }
            uint4* dst = (uint4*)(act.q + row * act.qstride + b * 32);
            dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
            dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
            act.d[row * act.dstride + b] = h2f(dh);
            act.s[row * act.sstride + b] = sum;
        }
        return;
    }
    int nb = act.cols / 256;
    for (int b = tid; b < nb; b += NT) {
        const float* x = v + b * 256;
        float max = 0.0f, amax = 0.0f;
        for (int j = 0; j < 256; j++) {
            float ax = fabsf(x[j]);
            if (ax > amax) { amax = ax; max = x[j]; }
        }
        // q(j) recomputed where it is needed: no private array
        const float iscale = amax == 0.0f ? 0.0f : -127.0f / max;
        auto qv = [&](int j) -> int {
            if (amax == 0.0f) return 0;
            int t = nearest_int(iscale * x[j]);
            return t < 127 ? t : 127;
        };
        act.d[row * act.dstride + b] = amax == 0.0f ? 0.0f : 1.0f / iscale;
        if (act.fmt == ACT_K4) {
            uint32_t* dst = (uint32_t*)(act.q + row * act.qstride + b * 256);
            for (int s = 0; s < 8; s++)
                for (int l = 0; l < 8; l++) {
                    uint32_t pk = 0;
                    for (int m = 0; m < 4; m++) pk |= (uint32_t)(qv(32 * s + l + 8 * m) & 0xFF) << (8 * m);
                    dst[s * 8 + l] = pk;
                }
            for (int j = 0; j < 16; j++) {
                int sum = 0;
                for (int i = 0; i < 16; i++) sum += qv(16 * j + i);
                act.s[row * act.sstride + b * 16 + j] = sum;
            }
        } else {
            uint32_t* dst = (uint32_t*)(act.q + row * act.qstride + (int64_t)b * 512);
            int* c = act.s + row * act.sstride + b * 128;
            for (int P = 0; P < 8; P++)
                for (int l = 0; l < 8; l++) {
                    int x0 = qv(32 * P + l), x1 = qv(32 * P + l + 8), x2 = qv(32 * P + 16 + l), x3 = qv(32 * P + 16 + l + 8);
                    dst[(P * 8 + l) * 2 + 0] = (uint32_t)(x0 & 0xFF) | ((uint32_t)(x1 & 0xFF) << 8);
                    dst[(P * 8 + l) * 2 + 1] = ((uint32_t)(x2 & 0xFF) << 16) | ((uint32_t)(x3 & 0xFF) << 24);
                    c[(2 * P) * 8 + l] = -32 * (x0 + x1);
                    c[(2 * P + 1) * 8 + l] = -32 * (x2 + x3);
                }
        }
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
    extern __shared__ float sbuf[];
    __shared__ double red[NT];
    const int t = blockIdx.x, tid = threadIdx.x;
    const float* xr = x + (int64_t)t * d;
    float scale = rms_scale_from_mean(mean_sq_cert<NT>(xr, d, red, flags), eps);
    float sc = 1.0f / (float)__dsqrt_rn((double)d);
    float* ri = router_in + (int64_t)t * d;
    for (int i = tid; i < d; i += NT) ri[i] = xr[i] * scale * sc * gis[i];
    int cols = act_gu.cols;
    for (int i = tid; i < cols; i += NT) sbuf[i] = i < d ? xr[i] * scale * pre2[i] : 0.0f;
    __syncthreads();
    quantize_row<NT>(sbuf, act_gu, t);
    if (ffn_norm) {
        __syncthreads();
        for (int i = tid; i < act_sh.cols; i += NT) sbuf[i] = i < d ? xr[i] * scale * ffn_norm[i] : 0.0f;
        __syncthreads();
        quantize_row<NT>(sbuf, act_sh, t);
    }
    if (tid == 0) xscale[t] = scale;
}

void launch_prologue(hipStream_t st, int T, int d, float eps, const float* x, const float* gis, const float* pre2,
                     const float* ffn_norm, float* router_in, float* xscale, Act act_gu, Act act_sh, int* flags)
{
    int cols = act_gu.cols > act_sh.cols ? act_gu.cols : act_sh.cols;
    if (cols < d) cols = d;
    launch(k_prologue<256>, dim3(T), dim3(256), (size_t)cols * sizeof(float), st, d, eps, x, gis, pre2,
                       ffn_norm, router_in, xscale, act_gu, act_sh, flags);
}

// ------------------------------------------------------------------------------ router logits
// logits[t][e] = sum_i W[e][i] * m[t][i] as the sequential float sum of GemmaCpu.cs:393-394: one lane
// per (t, e), the products rounded, then added in index order.  W is stored [d/4][E][4] so the 64
// lanes (experts) of a wave read 1 KB contiguous; m is wave-uniform.
template <int TB>
__global__ __launch_bounds__(64) void k_router_exact(int T, int d, int E, const float4* __restrict__ wt4,
                                                     const float* __restrict__ rin, float* __restrict__ logits)
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
}

// Many tokens: one wave per (64 experts, token) and no LDS, so the occupancy hides the load latency.
__global__ __launch_bounds__(64) void k_router_exact_wide(int d, int E, const float4* __restrict__ wt4,
                                                          const float* __restrict__ rin, float* __restrict__ logits)
{
    const int e = blockIdx.x * 64 + threadIdx.x, t = blockIdx.y;
    const int ee = e < E ? e : E - 1;
    const float4* w = wt4 + ee;
    const float4* m = (const float4*)(rin + (int64_t)t * d);
    float s = 0.0f;
    const int n4 = d / 4;
#pragma unroll 4
    for (int i = 0; i < n4; i++) {
        const float4 wv = w[(int64_t)i * E];
        const float4 mv = m[i];
        s += wv.x * mv.x;
        s += wv.y * mv.y;
        s += wv.z * mv.z;
        s += wv.w * mv.w;
    }
    if (e < E) logits[(int64_t)t * E + e] = s;
}

// Fewer tokens: each lane carries TB tokens' sequential chains (each in index order, as the
// reference): one read of W serves TB tokens and the independent chains fill the add latency.  The
// token rows of m sit in LDS; W streams in 32-element chunks, the next chunk's loads issued before the
// current chunk's adds.
void launch_router_exact(hipStream_t st, int T, int d, int E, const float* wt4, const float* rin, float* logits)
{
    const int gx = (E + 63) / 64;
    const float4* w = (const float4*)wt4;
    if (T >= 1024)
        launch(k_router_exact_wide, dim3(gx, T), dim3(64), 0, st, d, E, w, rin, logits);
    else if (T >= 128)
        launch(k_router_exact<2>, dim3(gx, (T + 1) / 2), dim3(64), (uint32_t)(2 * d * 4), st, T, d, E, w, rin, logits);
    else
        launch(k_router_exact<1>, dim3(gx, T), dim3(64), (uint32_t)(d * 4), st, T, d, E, w, rin, logits);
}

// ------------------------------------------------------------------------------ top-k and weights
// One wave per token.  k rounds of argmax with the lower expert index winning ties, the order of
// GemmaCpu.cs:400-405 (and the rank rule of KernelsMoe.RouterSelect, src/KernelsMoe.cs:64-78).
// Weights as GemmaCpu.cs:406-407,417: p_j = (float)exp((double)(l_j - l_0)), sum in double,
// w_j = (float)(p_j / sum) * down_scale[e_j]; rule 1 keeps the CPU's in-place sel[0] update.
__global__ __launch_bounds__(64) void k_topk(int E, int k, int rule, const float* __restrict__ logits,
                                             const float* __restrict__ ds, int* __restrict__ ids, float* __restrict__ wout)
{
    const int t = blockIdx.x, lane = threadIdx.x;
    __shared__ float sel[PHX_MAX_USED_DEV];
    __shared__ int sid[PHX_MAX_USED_DEV];
    float v[4];
    bool avail[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        int e = lane + 64 * q;
        avail[q] = e < E;
        v[q] = avail[q] ? logits[(int64_t)t * E + e] : 0.0f;
    }
    float key[4];
#pragma unroll
    for (int q = 0; q < 4; q++) key[q] = sel_key(v[q]);
    for (int j = 0; j < k; j++) {
        float bk = 0.0f, bv = 0.0f;
        int bi = -1;
#pragma unroll
        for (int q = 0; q < 4; q++)
            if (avail[q] && sel_beats(key[q], lane + 64 * q, bk, bi)) { bk = key[q]; bv = v[q]; bi = lane + 64 * q; }
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            float ok = __shfl_xor(bk, off, 64), ov = __shfl_xor(bv, off, 64);
            int oi = __shfl_xor(bi, off, 64);
            if (sel_beats(ok, oi, bk, bi)) { bk = ok; bv = ov; bi = oi; }
        }
        if (bi >= 0 && lane == (bi & 63)) avail[bi >> 6] = false;
        if (lane == 0) { sel[j] = bv; sid[j] = bi < 0 ? 0 : bi; }
    }
    __syncthreads();
    if (lane == 0) {
        float p[PHX_MAX_USED_DEV];
        double sum = 0.0;
        float top = sel[0];
        for (int j = 0; j < k; j++) {
            float pj = (float)exp((double)(sel[j] - top));
            if (rule == 1 && j == 0) top = pj;  // GemmaCpu.cs:407 overwrites sel[0] before later terms read it
            p[j] = pj;
            sum += (double)pj;
        }
        for (int j = 0; j < k; j++) {
            ids[(int64_t)t * k + j] = sid[j];
            wout[(int64_t)t * k + j] = (float)((double)p[j] / sum) * ds[sid[j]];
        }
    }
}

void launch_topk(hipStream_t st, int T, int E, int k, int rule, const float* logits, const float* ds, int* ids, float* w)
{
    launch(k_topk, dim3(T), dim3(64), 0, st, E, k, rule, logits, ds, ids, w);
}

// ------------------------------------------------------------------------------ dispatch
// Per-expert ascending assignment lists (the lists of KernelsMoe.Bucket, src/KernelsMoe.cs:281-330)
// as one stable counting sort in a single workgroup: per-chunk histograms, per-expert prefix over
// chunks, expert offsets, then every chunk places its assignments in order.  Also the work list of
// (expert, first list position, count <= A) tiles for the grouped kernels.
// chunks of the stable counting sort: at most 256 (one per thread) and at most 16,384 / E so the
// u16 histogram stays within 32 KB of LDS
__host__ __device__ inline int dispatch_chunks(int n, int E)
{
    int c = n < 256 ? (n > 0 ? n : 1) : 256;
    int cap = 16384 / (E > 0 ? E : 1);
    return c < cap ? c : (cap > 0 ? cap : 1);
}

__global__ __launch_bounds__(256) void k_dispatch(int n, int E, int A, const int* __restrict__ ids,
                                                  int* __restrict__ offsets, int* __restrict__ perm,
                                                  Tile* __restrict__ tiles, int* __restrict__ ntiles)
{
    extern __shared__ uint16_t hist[];  // [E][nch]
    __shared__ int tot[PHX_MAX_EXPERTS_DEV + 1], toff[PHX_MAX_EXPERTS_DEV + 1], tb[PHX_MAX_EXPERTS_DEV + 1];
    const int tid = threadIdx.x;
    const int nch = dispatch_chunks(n, E);
    const int cs = (n + nch - 1) / nch;
    for (int i = tid; i < E * nch; i += 256) hist[i] = 0;
    __syncthreads();
    const int a0 = tid * cs, a1 = min(n, a0 + cs);
    if (tid < nch)
        for (int a = a0; a < a1; a++) hist[clamp_id(ids[a], E) * nch + tid]++;
    __syncthreads();
    if (tid < E) {
        int run = 0;
        for (int c = 0; c < nch; c++) {
            int h = hist[tid * nch + c];
            hist[tid * nch + c] = (uint16_t)run;
            run += h;
        }
        tot[tid] = run;
    }
    __syncthreads();
    if (tid == 0) {
        int r = 0, tr = 0;
        for (int e = 0; e < E; e++) {
            toff[e] = r;
            r += tot[e];
            tb[e] = tr;
            tr += (tot[e] + A - 1) / A;
        }
        toff[E] = r;
        tb[E] = tr;
        *ntiles = tr;
    }
    __syncthreads();
    for (int e = tid; e <= E; e += 256) offsets[e] = toff[e];
    if (tid < nch)
        for (int a = a0; a < a1; a++) {
            int e = clamp_id(ids[a], E);
            int pos = toff[e] + hist[e * nch + tid];
            hist[e * nch + tid]++;
            perm[pos] = a;
        }
    if (tid < E) {
        int c = tot[tid], base = tb[tid];
        for (int s = 0; s * A < c; s++) {
            Tile tl;
            tl.e = tid;
            tl.start = toff[tid] + s * A;
            tl.cnt = min(A, c - s * A);
            tiles[base + s] = tl;
        }
    }
}

void launch_dispatch(hipStream_t st, int n, int E, int A, const int* ids, int* offsets, int* perm, Tile* tiles,
                     int* ntiles)
{
    int nch = dispatch_chunks(n, E);
    launch(k_dispatch, dim3(1), dim3(256), (size_t)E * nch * sizeof(uint16_t), st, n, E, A, ids, offsets,
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

// K-quant rows: DotK (src/CpuRefKQuants.cs:177-212) per (row, assignment): per super-block the eight
// integer lanes aux32[l] (element e contributes to lane e % 8), float lanes
// sums[l] += (d * yd) * aux32[l], the Q4_K min term sumf -= (dmin * yd) * sumi, finally sumf += sums[l].
template <int TYPE, int A>
__global__ __launch_bounds__(256) void k_grouped_k(GroupArgs g)
{
    const int tile = blockIdx.x;
    if (tile >= *g.ntiles) return;
    const Tile tl = g.tiles[tile];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rgi = blockIdx.y * 4 + wave;
    if (rgi >= g.rg) return;
    constexpr bool Q4K = TYPE == PHX_Q4_K_DEV;
    constexpr int PAY = Q4K ? 144 : 208;
    const uint8_t* wp = g.payload + tl.e * g.mat_pay + rgi * g.rg_pay + lane * PAY;
    const uint8_t* wsb = g.scale + tl.e * g.mat_sc + ((int64_t)rgi * g.nb * 64 + lane) * (Q4K ? 4 : 2);
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
        if (Q4K) {
            uint32_t dm = *(const uint32_t*)(wsb + (int64_t)b * 64 * 4);
            d = h2f(dm & 0xFFFF);
            dmin = h2f(dm >> 16);
        } else {
            d = h2f(*(const uint16_t*)(wsb + (int64_t)b * 64 * 2));
        }
        // unpacked weight dwords
        uint32_t v[64];
        int sc[16], mn[8];
        if (Q4K) {
#pragma unroll
            for (int w = 0; w < 32; w++) {
                v[2 * w] = wv[w] & 0x0F0F0F0Fu;
                v[2 * w + 1] = (wv[w] >> 4) & 0x0F0F0F0Fu;
            }
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
                if (Q4K) {
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
                if (Q4K) {
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

void launch_grouped(hipStream_t st, const QMat& w, Act act, const Tile* tiles, const int* ntiles, int max_tiles, int A,
                    const int* perm, int act_div, float* out0, float* out1, int split, int out_stride)
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
    dim3 grid(max_tiles, (w.rg + 3) / 4);
    if (A != 4) A = 4;  // the tile size the dispatch used; one instantiation for now
    switch (w.type) {
    case PHX_Q4_0_DEV: launch((k_grouped_q<PHX_Q4_0_DEV, 4>), grid, dim3(256), 0, st, g); break;
    case PHX_Q8_0_DEV: launch((k_grouped_q<PHX_Q8_0_DEV, 4>), grid, dim3(256), 0, st, g); break;
    case PHX_Q4_K_DEV: launch((k_grouped_k<PHX_Q4_K_DEV, 4>), grid, dim3(256), 0, st, g); break;
    case PHX_Q6_K_DEV: launch((k_grouped_k<PHX_Q6_K_DEV, 4>), grid, dim3(256), 0, st, g); break;
    }
}

// ------------------------------------------------------------------------------ GELU-gated requant
// Per assignment row: e = gelu(g) * u (src/GemmaCpu.cs:415), zero padding up to act.cols, then the
// activation quantizer of the down weights (Q8_0 or Q8_K on entry to the down MatVec).
__global__ __launch_bounds__(256) void k_requant(int nf, const float* __restrict__ g, const float* __restrict__ u,
                                                 const float* __restrict__ tab, Act act)
{
    extern __shared__ float sbuf[];
    const int64_t r = blockIdx.x;
    const int tid = threadIdx.x;
    for (int i = tid; i < act.cols; i += 256)
        sbuf[i] = i < nf ? gelu_ref(g[r * nf + i], tab) * u[r * nf + i] : 0.0f;
    __syncthreads();
    quantize_row<256>(sbuf, act, r);
}

void launch_requant(hipStream_t st, int rows, int nf, const float* g, const float* u, const float* tab, Act act)
{
    launch(k_requant, dim3(rows), dim3(256), (size_t)act.cols * sizeof(float), st, nf, g, u, tab, act);
}

// ------------------------------------------------------------------------------ combine, norms, residual
// Per token: acc = sum_j yd[t*k+j] * w_j in rank order (src/GemmaCpu.cs:418, each term rounded then
// added), out = rmsnorm(shared) * post1 + rmsnorm(acc) * post2 (src/GemmaCpu.cs:384,420-421), and
// optionally x += rmsnorm(out) * post_ffw_norm (src/GemmaCpu.cs:355-356).
__global__ __launch_bounds__(256) void k_combine(int d, int k, float eps, const float* __restrict__ yd,
                                                 const float* __restrict__ w, const float* __restrict__ shared,
                                                 const float* __restrict__ post1, const float* __restrict__ post2,
                                                 float* __restrict__ out, float* __restrict__ xres,
                                                 const float* __restrict__ post_ffw, int* flags)
{
    extern __shared__ float sbuf[];  // [2][d]
    __shared__ double red[256];
    const int t = blockIdx.x, tid = threadIdx.x;
    float* acc = sbuf;
    float* o = sbuf + d;
    for (int i = tid; i < d; i += 256) {
        float a = 0.0f;
        for (int j = 0; j < k; j++) a += yd[((int64_t)t * k + j) * d + i] * w[(int64_t)t * k + j];
        acc[i] = a;
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

void launch_combine(hipStream_t st, int T, int d, int k, float eps, const float* yd, const float* w, const float* shared,
                    const float* post1, const float* post2, float* out, float* xres, const float* post_ffw, int* flags)
{
    launch(k_combine, dim3(T), dim3(256), (size_t)2 * d * sizeof(float), st, d, k, eps, yd, w, shared, post1,
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

// ------------------------------------------------------------------------------ arithmetic self-test
__global__ void k_selftest(int op, int n, const float* __restrict__ a, const float* __restrict__ b, float* __restrict__ out,
                           const float* __restrict__ tab)
{
    int i = blockIdx.x * blockDim.x + threadIdx.x;
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

}  // namespace phx
