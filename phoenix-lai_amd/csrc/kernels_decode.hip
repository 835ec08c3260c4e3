// Decode-shaped MoE FFN kernels (a few tokens, T <= 16; Q4_0 / Q8_0 weights): four launches per layer.
//   k_dec_route    router logits with certified error bounds, one workgroup per (token, expert), and the
//                  Q8_0 expert and shared-FFN inputs (each workgroup quantizes its share of the
//                  token's 32-blocks)
//   k_dec_gu       at most one workgroup per CU, each over a strided share of the units: first the
//                  dense shared FFN's (token pair, row group) gate|up units, then the routed experts'
//                  (tile, row group) units with the gelu(g) * u Q8_0 epilogue.  Before its first expert
//                  unit a workgroup selects the top-k from the router's bounds (exact fallback when the
//                  order cannot be certified) and forms the expert tiles; the last workgroup writes
//                  the routing outputs
//   k_dec_down     (tile, row groups) of the routed experts' down products; beside them, the shared
//                  FFN's down product
//   k_dec_combine  per token: the rank-ordered combine, the two branch norms, the optional residual
// Arithmetic follows the reference CPU path (src/GemmaCpu.cs:376-422): integer block sums, the float
// block chain sum += (float)isum * (d_w * d_x) in block order (src/CpuRefGemma.cs:27-36,
// src/CpuRef.cs:106-115), the rank-ordered combine (GemmaCpu.cs:417-418) and RmsNorm's double sums of
// squares (src/CpuRef.cs:183-191) reproduced through certified bounds.  The router logits are the one
// quantity certified rather than replayed (k_dec_route).
//
// Work layout: a row group (64 rows, lane = row) is one workgroup of ceil(nb / 8) waves, wave w
// holding blocks 8w..8w+7 of its lane's row.  Every wave issues its 8 payload loads (16 B per lane, a
// 1 KB contiguous span per instruction) and one 16 B load of the 8 blocks' fp16 scales before it
// waits on any of them; the small activation loads are issued before the weights, so the first wait
// is for them alone.  Block indices past the row end are clamped, never branched around.  These
// kernels are bound by latency and by the CU's issue rate, so per-thread work is sized at compile time
// (no masked slots) and reductions use DPP.
#include <algorithm>

#include "device_common.h"

namespace phx {


constexpr int DMAXNB = 128;  // blocks of 32 per row: K <= 4096
constexpr int DROWS = 2;     // assignments (expert tiles) or tokens (shared FFN) per workgroup
constexpr int DBPW = 8;      // blocks per wave

template <int TYPE>
struct DecCfg {
    static constexpr int PAY = TYPE == PHX_Q4_0_DEV ? 16 : 32;  // payload bytes per block
    static constexpr int NC = PAY / 16;                         // 16 B loads per block
};

// decode-layout view of one matrix stack (QMat): row group rg of matrix m at pay + m * mat_pay +
// rg * rg_pay holds the blocks [b][64][PAY], then at sc_off the scale groups [b/8][64][8] fp16
struct MatD {
    const uint8_t* pay;
    int64_t mat_pay;  // bytes per matrix
    int64_t rg_pay;   // bytes per row group
    int64_t sc_off;   // scale groups within a row group
    int rg, nb, nb8, rows;
};

// Q8_0 activation rows in LDS: q as 8 dwords per block, the fp16 scale value, the block sum
struct ActL {
    int q[DMAXNB * 8];
    float d[DMAXNB];
    int s[DMAXNB];
};

struct DecArgs {
    int T, d, E, k, nf, nff, rule, max_tiles;
    int seq;              // position in a captured stack (clock-stamp slot of the instrumented build)
    float eps;
    const float* x;       // [T][d]
    const float* xscale;  // [T] the rows' rms scales when the prologue formed them (else null)
    const float* W;       // [E][d] router (ffn_gate_inp.weight)
    const float* gis;     // ffn_gate_inp.scale
    const float* ds;      // ffn_down_exps.scale
    const float* pre2;    // pre_ffw_norm_2
    const float* post1;   // post_ffw_norm_1
    const float* post2;   // post_ffw_norm_2
    const float* fnorm;   // ffn_norm (shared FFN input)
    const float* post_ffw;
    MatD gu, dn, sgu, sdn;  // sgu.rg == 0: no shared FFN computed
    Act agu;              // packed Q8_0 expert input rows [T] (k_dec_route writes, k_dec_gu reads)
    Act ash;              // packed Q8_0 shared-FFN input rows [T]
    int rpw;              // k_dec_down: expert row groups per workgroup
    double* Lb;           // [T][E] certified logits (double sums)
    double* Bb;           // [T][E] their error bounds
    uint4* kb;            // [T][E] selection keys: rank key, lower end, upper end, finite (route_wg)
    int* cbad;            // [1 + T]: the count, then the tokens k_cert_select leaves to the exact chains
    int* ids;             // [T][k]
    float* w;             // [T][k]
    float* logits;        // [T][E]
    int* offsets;         // [E + 1]
    int* perm;            // [T * k]
    DecTile* tiles;       // [max_tiles] (e = -1 past the last tile)
    float* g;             // [T*k][nf] gate products
    float* u;             // [T*k][nf] up products
    Act adn;              // Q8_0 of gelu(g) * u: the down input, [T*k][nf]
    float* yd;            // [T*k][d] down products
    float* shg;           // [T][nff]
    float* shu;
    Act asd;              // Q8_0 of the shared gelu(g) * u, [T][nff]
    float* shout;         // [T][d] shared branch (the shared FFN's output, or the given one), or null
    float* out;           // [T][d]
    float* xres;          // x updated in place with the residual, or null
    const float* xin;     // with xres: the residual's source rows when not xres itself (or null)
    const float* gelu_tab;
    int* flags;           // [0] norm fallbacks, [1] router fallbacks
};

// ------------------------------------------------------------------------------ helpers


// Mean of squares of a row (RmsNorm's (float)(sum / n), sum the sequential double sum of x_i^2,
// src/CpuRef.cs:186-188) from per-thread partial double sums `s` over disjoint elements.  Any order of
// summing n non-negative terms is within (n + 64) * 2^-52 * sum of the sequential sum (the summation
// depth here is far below 64); when both ends of that interval give the same float the result is the
// reference's, otherwise thread 0 re-sums sequentially (rare; counted in *fallbacks when non-null).
// Workgroup-level: every thread calls it; red holds blockDim.x / 64 + 1 doubles.  TRAIL: a closing
// barrier, for callers that reuse red right after.  WAVE: the sequential sum by wave 0
// (seq_sum_sq_wave), else by thread 0 alone (for kernels whose registers are tight).
template <bool TRAIL = true, bool WAVE = true>
__device__ float wg_mean_sq(double s, const float* xr, int n, double* red, int* fallbacks)
{
    const int tid = threadIdx.x, lane = tid & 63, nw = blockDim.x >> 6;
    s = wave_sum_dpp(s);
    if (lane == 0) red[tid >> 6] = s;
    __syncthreads();
    const double S = wave_sum_dpp(lane < nw ? red[lane] : 0.0);  // the wave totals in a fixed tree order
    const double B = ((double)n + 64.0) * 0x1p-52 * S;
    float lo, hi;
    mean_ends(S, B, 1.0 / (double)n, &lo, &hi);
    float mean = lo;
    if (lo != hi) {  // uniform: every thread formed the same S
        if (WAVE ? tid < 64 : tid == 0) {
            double q = 0.0;
            if (WAVE) q = seq_sum_sq_wave(xr, n);
            else
                for (int i = 0; i < n; i++) q += (double)xr[i] * (double)xr[i];
            if (tid == 0) {
                red[nw] = q;
                if (fallbacks) atomicAdd(fallbacks, 1);
            }
        }
        __syncthreads();
        mean = (float)(red[nw] / (double)n);
    }
    if (TRAIL) __syncthreads();  // red is reused by the next call
    return mean;
}

// The means of squares of two rows in one reduction pass, each by the rule of wg_mean_sq (x1 may be
// null when s1 is zero everywhere).  red holds 2 * (blockDim.x / 64 + 1) doubles.
template <bool TRAIL = true>
__device__ void wg_mean_sq2(double s0, double s1, const float* x0, const float* x1, int n, double* red,
                            int* fallbacks, float* m0, float* m1)
{
    const int tid = threadIdx.x, lane = tid & 63, nw = blockDim.x >> 6;
    double* red1 = red + nw + 1;
    s0 = wave_sum_dpp(s0);
    s1 = wave_sum_dpp(s1);
    if (lane == 0) {
        red[tid >> 6] = s0;
        red1[tid >> 6] = s1;
    }
    __syncthreads();
    const double S0 = wave_sum_dpp(lane < nw ? red[lane] : 0.0);
    const double S1 = wave_sum_dpp(lane < nw ? red1[lane] : 0.0);
    const double B0 = ((double)n + 64.0) * 0x1p-52 * S0, B1 = ((double)n + 64.0) * 0x1p-52 * S1;
    const double rn = 1.0 / (double)n;
    float lo0, hi0, lo1, hi1;
    mean_ends(S0, B0, rn, &lo0, &hi0);
    mean_ends(S1, B1, rn, &lo1, &hi1);
    if (lo0 != hi0 || lo1 != hi1) {  // uniform: every thread formed the same sums
        if (tid < 64) {
            if (lo0 != hi0) {
                const double q = seq_sum_sq_wave(x0, n);
                if (tid == 0) {
                    red[nw] = q;
                    if (fallbacks) atomicAdd(fallbacks, 1);
                }
            }
            if (lo1 != hi1 && x1) {
                const double q = seq_sum_sq_wave(x1, n);
                if (tid == 0) {
                    red1[nw] = q;
                    if (fallbacks) atomicAdd(fallbacks, 1);
                }
            }
        }
        __syncthreads();
        if (lo0 != hi0) lo0 = (float)(red[nw] / (double)n);
        if (lo1 != hi1 && x1) lo1 = (float)(red1[nw] / (double)n);
    }
    *m0 = lo0;
    *m1 = lo1;
    if (TRAIL) __syncthreads();  // red is reused by the next call
}

// The Q8_0 input rows of a gate|up workgroup: n_i = (x_i * rinv) * nw_i (src/GemmaCpu.cs:409 with
// CpuRef.RmsNorm, src/CpuRef.cs:183-191; the shared FFN: ffn_norm, :349), rinv the token's RmsNorm
// scale, quantized per 32-block into act[r].  8-lane group g takes block g (the workgroup has at least
// 8 * nb threads).  quant_issue loads the values (before the weight loads); quant_finish forms the rows.
struct QIn {
    float4 x0, x1, nw;
};

__device__ __forceinline__ void quant_issue(QIn& in, const float* x, int tok0, int tok1, const float* nw, int d)
{
    const int tid = threadIdx.x, nb = d / 32;
    const int i = min(tid >> 3, nb - 1) * 8 + (tid & 7);
    in.nw = ((const float4*)nw)[i];
    in.x0 = ((const float4*)(x + (int64_t)tok0 * d))[i];
    in.x1 = ((const float4*)(x + (int64_t)tok1 * d))[i];  // tok1 == tok0 for one row: no branch
}

__device__ __forceinline__ void quant_row(float4 xv, float4 nwv, const float* xr, int d, float eps, ActL& act,
                                          double* red, int* fallbacks)
{
    const int tid = threadIdx.x, b = tid >> 3, l8 = tid & 7, nb = d / 32;
    double s = 0.0;
    if (b < nb)
        s = ((double)xv.x * (double)xv.x + (double)xv.y * (double)xv.y) +
            ((double)xv.z * (double)xv.z + (double)xv.w * (double)xv.w);
    const float rinv = rms_scale_from_mean(wg_mean_sq(s, xr, d, red, fallbacks), eps);
    const float4 v = make_float4((xv.x * rinv) * nwv.x, (xv.y * rinv) * nwv.y, (xv.z * rinv) * nwv.z,
                                 (xv.w * rinv) * nwv.w);
    float dval;
    int sum;
    const int qw = q8_0_oct(v, &dval, &sum);
    if (b < nb) {
        act.q[b * 8 + l8] = qw;
        if (l8 == 0) {
            act.d[b] = dval;
            act.s[b] = sum;
        }
    }
}

__device__ __forceinline__ void quant_finish(const QIn& in, const float* x, int tok0, int tok1, int cnt, int d, float eps,
                                             ActL* act, double* red, int* fallbacks)
{
    quant_row(in.x0, in.nw, x + (int64_t)tok0 * d, d, eps, act[0], red, fallbacks);
    if (cnt > 1) quant_row(in.x1, in.nw, x + (int64_t)tok1 * d, d, eps, act[1], red, fallbacks);
}

// Q8_0 rows of a packed global activation buffer into LDS (nb blocks each): act_issue loads them into
// registers (before the weight loads), act_store writes them to LDS.  A packed global row is 10 * nb
// contiguous dwords: q (8 nb), d (nb), s (nb) (the decode path's Act buffers, see the runtime); an ActL
// row holds the same at fixed offsets.  The workgroup has at least 8 * nb threads, so two dwords per
// thread and row cover 10 * nb.
struct ActIn {
    int v[DROWS][2];
};

__device__ __forceinline__ const int* act_src(const Act& src, int64_t row, int nb, int i)
{
    return (const int*)(src.q + row * src.qstride) + min(i, 10 * nb - 1);
}

__device__ __forceinline__ int act_dst(int nb, int i)  // dword index in an ActL row
{
    return i < 8 * nb ? i : i < 9 * nb ? 8 * DMAXNB + (i - 8 * nb) : 9 * DMAXNB + (i - 9 * nb);
}

__device__ __forceinline__ void act_issue(ActIn& in, const Act& src, int64_t row0, int64_t row1, int cnt, int nb)
{
    const int tid = threadIdx.x, nt = blockDim.x;
#pragma unroll
    for (int c = 0; c < 2; c++) {
        const int i = min(tid + nt * c, 10 * nb - 1);
        in.v[0][c] = *act_src(src, row0, nb, i);
        in.v[1][c] = *act_src(src, row1, nb, i);  // row1 == row0 for one row: no branch
    }
}

__device__ __forceinline__ void act_store(const ActIn& in, int cnt, int nb, ActL* act)
{
    const int tid = threadIdx.x, nt = blockDim.x;
#pragma unroll
    for (int r = 0; r < DROWS; r++) {
        if (r < cnt) {
#pragma unroll
            for (int c = 0; c < 2; c++) {
                const int i = tid + nt * c;
                if (i < 10 * nb) ((int*)&act[r])[act_dst(nb, i)] = in.v[r][c];
            }
        }
    }
}

// Weight registers of one wave: blocks 8w..8w+7 of the lane's row (indices clamped to the row) and
// their 8 fp16 scales.
template <int TYPE>
struct WRegs {
    uint4 p[DBPW][DecCfg<TYPE>::NC];
    uint4 s;
};

template <int TYPE>
__device__ __forceinline__ void load_w(const MatD& M, int e, int rgi, int wave, int lane, WRegs<TYPE>& W)
{
    constexpr int PAY = DecCfg<TYPE>::PAY, NC = DecCfg<TYPE>::NC;
    // unconditional: a wave past the row reloads the row's last blocks (no branch around the loads, so
    // the compiler's wait counts stay exact)
    const int b0 = min(wave * DBPW, (M.nb8 - 1) * DBPW);
    const uint8_t* rgp = M.pay + (int64_t)e * M.mat_pay + (int64_t)rgi * M.rg_pay;
    const uint8_t* p = rgp + lane * PAY;
#pragma unroll
    for (int j = 0; j < DBPW; j++) {
        const int b = min(b0 + j, M.nb - 1);
#pragma unroll
        for (int c = 0; c < NC; c++) W.p[j][c] = *(const uint4*)(p + (int64_t)b * 64 * PAY + 16 * c);
    }
    W.s = *(const uint4*)(rgp + M.sc_off + ((b0 / DBPW) * 64 + lane) * 16);
}

// fp16 scale bits of block j of a WRegs
template <int TYPE>
__device__ __forceinline__ uint32_t w_scale(const WRegs<TYPE>& W, int j)
{
    const int h = j / 2;
    const uint32_t wd = h == 0 ? W.s.x : h == 1 ? W.s.y : h == 2 ? W.s.z : W.s.w;
    return (j & 1) ? wd >> 16 : wd & 0xFFFFu;
}

// The reference block term (float)isum * (d_w * d_x) of block j of W against activation block b.
template <int TYPE>
__device__ __forceinline__ float blk_term(const WRegs<TYPE>& W, int j, const ActL& a, int b)
{
    const int4 xa = *(const int4*)&a.q[b * 8];
    const int4 xb = *(const int4*)&a.q[b * 8 + 4];
    int isum = 0;
    if (TYPE == PHX_Q4_0_DEV) {
        const uint4 w = W.p[j][0];
        // low nibbles: elements 0..15 (x words 0..3); high nibbles: elements 16..31 (x words 4..7)
        isum = __builtin_amdgcn_sdot4((int)(w.x & 0x0F0F0F0Fu), xa.x, isum, false);
        isum = __builtin_amdgcn_sdot4((int)(w.y & 0x0F0F0F0Fu), xa.y, isum, false);
        isum = __builtin_amdgcn_sdot4((int)(w.z & 0x0F0F0F0Fu), xa.z, isum, false);
        isum = __builtin_amdgcn_sdot4((int)(w.w & 0x0F0F0F0Fu), xa.w, isum, false);
        isum = __builtin_amdgcn_sdot4((int)((w.x >> 4) & 0x0F0F0F0Fu), xb.x, isum, false);
        isum = __builtin_amdgcn_sdot4((int)((w.y >> 4) & 0x0F0F0F0Fu), xb.y, isum, false);
        isum = __builtin_amdgcn_sdot4((int)((w.z >> 4) & 0x0F0F0F0Fu), xb.z, isum, false);
        isum = __builtin_amdgcn_sdot4((int)((w.w >> 4) & 0x0F0F0F0Fu), xb.w, isum, false);
        isum -= 8 * a.s[b];
    } else {
        const uint4 w0 = W.p[j][0], w1 = W.p[j][DecCfg<TYPE>::NC - 1];
        isum = __builtin_amdgcn_sdot4((int)w0.x, xa.x, isum, false);
        isum = __builtin_amdgcn_sdot4((int)w0.y, xa.y, isum, false);
        isum = __builtin_amdgcn_sdot4((int)w0.z, xa.z, isum, false);
        isum = __builtin_amdgcn_sdot4((int)w0.w, xa.w, isum, false);
        isum = __builtin_amdgcn_sdot4((int)w1.x, xb.x, isum, false);
        isum = __builtin_amdgcn_sdot4((int)w1.y, xb.y, isum, false);
        isum = __builtin_amdgcn_sdot4((int)w1.z, xb.z, isum, false);
        isum = __builtin_amdgcn_sdot4((int)w1.w, xb.w, isum, false);
    }
    const float dd = h2f(w_scale(W, j)) * a.d[b];
    return (float)isum * dd;
}

// One row group for cnt <= DROWS activation rows, computed by the waves wl = 0, 1, ... of the group
// (wave wl holds blocks 8 wl..8 wl+7): every wave's block terms into LDS (terms[r][b][lane], row stride
// nb), a workgroup barrier, then wave wl = r adds row r's terms in block order.  Returns the chain value
// in waves wl < cnt (0 elsewhere).  Every wave of the workgroup calls it once (one barrier).
template <int TYPE>
__device__ float rowgroup_chain(const WRegs<TYPE>& W, int wl, int nb, const ActL* act, int cnt, float* terms)
{
    const int lane = threadIdx.x & 63, b0 = wl * DBPW;
    if (b0 < nb) {  // uniform per wave
        for (int r = 0; r < cnt; r++) {
#pragma unroll
            for (int j = 0; j < DBPW; j++) {
                const int b = min(b0 + j, nb - 1);
                const float t = blk_term(W, j, act[r], b);
                if (b0 + j < nb) terms[(r * nb + b0 + j) * 64 + lane] = t;
            }
        }
    }
    __syncthreads();
    float S = 0.0f;
    if (wl < cnt) {
        const float* tr = terms + wl * nb * 64 + lane;
        int b = 0;
        for (; b + 8 <= nb; b += 8) {
            float t[8];
#pragma unroll
            for (int i = 0; i < 8; i++) t[i] = tr[(b + i) * 64];
#pragma unroll
            for (int i = 0; i < 8; i++) S += t[i];
        }
        for (; b < nb; b++) S += tr[b * 64];
    }
    return S;
}

// gate|up epilogue of a paired row group (lanes 0-31 gate rows 32 rgi + l, lanes 32-63 the matching
// up rows): g and u to the debug outputs, e = gelu(g) * u (src/GemmaCpu.cs:415) quantized to the
// Q8_0 block rgi of the down input row (src/CpuRef.cs:49-62).
__device__ __forceinline__ void gu_epilogue(float S, int rgi, int split, int64_t orow, float* g, float* u, const Act& o,
                                            const float* gelu_tab)
{
    const int lane = threadIdx.x & 63;
    const int jj = rgi * 32 + (lane & 31);
    const float uv = __shfl_down(S, 32, 64);
    if (jj < split) {
        if (lane < 32) g[orow * split + jj] = S;
        else u[orow * split + jj] = S;
    }
    const float ev = lane < 32 ? gelu_ref(S, gelu_tab) * uv : 0.0f;
    float dval;
    int sum;
    const int q = q8_0_half(ev, &dval, &sum);
    if (lane < 32) {
        o.q[orow * o.qstride + jj] = (int8_t)q;
        if (lane == 0) {
            o.d[orow * o.dstride + rgi] = dval;
            o.s[orow * o.sstride + rgi] = sum;
        }
    }
}

// ------------------------------------------------------------------------------ combine of a token
// The layer's output for token t by a whole workgroup whose threads hold CQ float4 columns each
// (CQ * 4 * blockDim.x >= d): acc = sum_j w_j * yd_j in rank order (src/GemmaCpu.cs:417-418, each
// term rounded then added), out = rmsnorm(shared) * post1 + rmsnorm(acc) * post2 (src/GemmaCpu.cs:384,
// 420-421), x_new = x + rmsnorm(out) * post_ffw_norm (src/GemmaCpu.cs:355-356), the same expressions
// as k_dec_combine.  Every load is issued in one round into registers (the caller's occupancy is set
// by its LDS, so the registers are free); x_new lands in sx (LDS, [d]) and this thread's float4s of it
// in xkeep; with leader, out and x_new also go to p.out and p.xres (x read from p.xin).  sacc and so:
// LDS [d] each; red: 3 * (blockDim.x / 64 + 1) doubles.  No barrier after the last pass: the caller's
// next barrier publishes sx.
// What the combine of a layer reads and writes (a small kernel argument of the fused router)
struct CombArgs {
    int d, k, seq;
    float eps;
    const float *w, *yd, *shout, *post1, *post2, *post_ffw, *xin;
    float *out, *xres;
    int* flags;
};

template <int CQ, class F>
__device__ __forceinline__ void combine_into(const CombArgs& p, int t, float* sx, float* sacc, float* so, double* red,
                                             bool leader, F&& after_issue, float4* xkeep)
{
    constexpr int RG = CQ <= 3 ? 8 : 4;  // ranks per load round (register budget)
    const int tid = threadIdx.x, NT = blockDim.x, d = p.d, k = p.k, n4 = d / 4;
    const float4* sh4 = p.shout ? (const float4*)(p.shout + (int64_t)t * d) : nullptr;
    const float4 z4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    int ix[CQ];
    float4 acc[CQ], shv[CQ], p1[CQ], p2[CQ], xv[CQ], pf[CQ];
#pragma unroll
    for (int q = 0; q < CQ; q++) {
        ix[q] = min(tid + q * NT, n4 - 1);
        acc[q] = z4;
    }
    // pass 1: every load of the token in one round (ranks RG at a time), acc in rank order
    for (int j0 = 0; j0 < k; j0 += RG) {
        float4 yv[CQ][RG];
        float wj[RG];
#pragma unroll
        for (int jj = 0; jj < RG; jj++) wj[jj] = p.w[(int64_t)t * k + min(j0 + jj, k - 1)];
#pragma unroll
        for (int q = 0; q < CQ; q++)
#pragma unroll
            for (int jj = 0; jj < RG; jj++)
                yv[q][jj] = ((const float4*)(p.yd + ((int64_t)t * k + min(j0 + jj, k - 1)) * d))[ix[q]];
        if (j0 == 0) {
#pragma unroll
            for (int q = 0; q < CQ; q++) {
                shv[q] = sh4 ? sh4[ix[q]] : z4;
                p1[q] = ((const float4*)p.post1)[ix[q]];
                p2[q] = ((const float4*)p.post2)[ix[q]];
                xv[q] = ((const float4*)(p.xin + (int64_t)t * d))[ix[q]];
                pf[q] = ((const float4*)p.post_ffw)[ix[q]];
            }
            // the caller's own loads go out behind these (the first use waits for these alone)
            __builtin_amdgcn_sched_barrier(0);
            after_issue();
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int q = 0; q < CQ; q++)
#pragma unroll
            for (int jj = 0; jj < RG; jj++)
                if (j0 + jj < k) {
                    acc[q].x += yv[q][jj].x * wj[jj];
                    acc[q].y += yv[q][jj].y * wj[jj];
                    acc[q].z += yv[q][jj].z * wj[jj];
                    acc[q].w += yv[q][jj].w * wj[jj];
                }
    }
    TL_STAMP(p.seq, 3, 4);
    double s2 = 0.0, s1 = 0.0;
#pragma unroll
    for (int q = 0; q < CQ; q++)
        if (tid + q * NT < n4) {
            ((float4*)sacc)[tid + q * NT] = acc[q];
            s2 += (double)acc[q].x * (double)acc[q].x + (double)acc[q].y * (double)acc[q].y;
            s2 += (double)acc[q].z * (double)acc[q].z + (double)acc[q].w * (double)acc[q].w;
            s1 += (double)shv[q].x * (double)shv[q].x + (double)shv[q].y * (double)shv[q].y;
            s1 += (double)shv[q].z * (double)shv[q].z + (double)shv[q].w * (double)shv[q].w;
        }
    // (the reductions' own barriers publish sacc and so to their sequential fallbacks; the two use
    // separate parts of red, so neither needs a closing barrier)
    float m2, m1;
    wg_mean_sq2<false>(s2, s1, sacc, sh4 ? (const float*)sh4 : nullptr, d, red, leader ? p.flags : nullptr, &m2, &m1);
    const float sc2 = rms_scale_from_mean(m2, p.eps);
    const float sc1 = sh4 ? rms_scale_from_mean(m1, p.eps) : 0.0f;
    TL_STAMP(p.seq, 3, 5);
    // pass 2: out = rmsnorm(shared) * post1 + rmsnorm(acc) * post2 and its sum of squares
    float4 ov[CQ];
    double s3 = 0.0;
#pragma unroll
    for (int q = 0; q < CQ; q++) {
        ov[q].x = (sh4 ? shv[q].x * sc1 * p1[q].x : 0.0f) + acc[q].x * sc2 * p2[q].x;
        ov[q].y = (sh4 ? shv[q].y * sc1 * p1[q].y : 0.0f) + acc[q].y * sc2 * p2[q].y;
        ov[q].z = (sh4 ? shv[q].z * sc1 * p1[q].z : 0.0f) + acc[q].z * sc2 * p2[q].z;
        ov[q].w = (sh4 ? shv[q].w * sc1 * p1[q].w : 0.0f) + acc[q].w * sc2 * p2[q].w;
        const int i4 = tid + q * NT;
        if (i4 < n4) {
            ((float4*)so)[i4] = ov[q];
            if (leader) ((float4*)(p.out + (int64_t)t * d))[i4] = ov[q];
            s3 += (double)ov[q].x * (double)ov[q].x + (double)ov[q].y * (double)ov[q].y;
            s3 += (double)ov[q].z * (double)ov[q].z + (double)ov[q].w * (double)ov[q].w;
        }
    }
    const float sc3 =
        rms_scale_from_mean(wg_mean_sq<false>(s3, so, d, red + 2 * (NT / 64 + 1), leader ? p.flags : nullptr), p.eps);
    TL_STAMP(p.seq, 3, 6);
    // pass 3: x_new = x + rmsnorm(out) * post_ffw_norm
#pragma unroll
    for (int q = 0; q < CQ; q++) {
        const int i4 = tid + q * NT;
        const float4 xn = make_float4(xv[q].x + ov[q].x * sc3 * pf[q].x, xv[q].y + ov[q].y * sc3 * pf[q].y,
                                      xv[q].z + ov[q].z * sc3 * pf[q].z, xv[q].w + ov[q].w * sc3 * pf[q].w);
        xkeep[q] = xn;
        if (i4 < n4) {
            ((float4*)sx)[i4] = xn;
            if (leader) ((float4*)(p.xres + (int64_t)t * d))[i4] = xn;
        }
    }
}

__device__ __forceinline__ float f32_down(double v)  // the largest float <= v
{
    const float f = (float)v;
    if (!((double)f > v)) return f;
    if (f == 0.0f) return -__uint_as_float(1u);  // below zero: minus the smallest subnormal
    const unsigned b = __float_as_uint(f);
    return __uint_as_float(f > 0.0f ? b - 1u : b + 1u);
}

__device__ __forceinline__ float f32_up(double v)  // the smallest float >= v
{
    const float f = (float)v;
    if (!((double)f < v)) return f;
    if (f == 0.0f) return __uint_as_float(1u);
    const unsigned b = __float_as_uint(f);
    return __uint_as_float(f > 0.0f ? b + 1u : b - 1u);
}

// expert e's selection key and interval ends for the gate|up launch's ranking (see wave_topk)
__device__ __forceinline__ uint4 sel_key(double L, double B, int e)
{
    const bool f = isfinite(L) && isfinite(B);
    return make_uint4((sortable_f32((float)L) & ~0xFFu) | (unsigned)(255 - e), f ? sortable_f32(f32_down(L - B)) : 0u,
                      f ? sortable_f32(f32_up(L + B)) : 0xFFFFFFFFu, f ? 1u : 0u);
}

// ------------------------------------------------------------------------------ k_dec_route
// One workgroup of d / 4 threads per (token t, expert e) (d % 256 == 0, d <= 4096: whole waves, at most
// 16); thread i holds the four consecutive elements 4i..4i+3 (x_t, the router scale and W[e] staged in
// LDS by one direct global -> LDS load per thread and row).  Many short per-thread chains rather than
// four waves of long ones: a SIMD with one wave issues an instruction only every ~8.7 cycles.  The reference logit is the sequential float sum
// of the rounded products p_i = fl(W[e][i] * m_i), m_i = ((x_i * rinv) * sc) * s_i
// (src/GemmaCpu.cs:389-395).  The workgroup forms the same p_i, sums them in double (L, from a scan of
// the chunk sums), and bounds the reference's accumulated rounding by
//   |S_ref - L| <= 2^-24 * sum_k |S_k| * 1.001 + 2^-45 * sum_i |p_i|,
// S_k the prefix sums; sum_k |S_k| and sum_i |p_i| are accumulated in float and enlarged by 2^-10 (far
// above their float rounding, so the bound still holds).  k_dec_gu ranks the experts by L and
// certifies the order from these intervals.  The workgroup also writes the Q8_0 expert input
// n = (x * rinv) * pre_ffw_norm_2 (src/GemmaCpu.cs:409) and the shared-FFN input (x * rinv) * ffn_norm
// (:349) of the 32-blocks b with b % E == e, one 8-lane group per block.
constexpr int RT_PER = 4, RT_MAXW = 16;  // elements per thread, waves per workgroup at most
__host__ __device__ inline int route_threads(int d) { return d / RT_PER; }

// the matrix-core kernels' copy of a Q8_0 activation dword (four integers as exact fp16, or folded with
// the block scale dval for the tolerance mode), for the general path's rows when it routes through this
// kernel
__device__ __forceinline__ void store_qh(const Act& act, int t, int b, int l8, int qw, float dval)
{
    *(uint2*)(act.qh + (int64_t)t * act.qhstride + 32 * b + 4 * l8) = act.fold ? fold_q4(qw, dval) : int_q4(qw);
}

template <int PER, bool FUSED>
__device__ __forceinline__ void route_wg(const DecArgs& a, int t, int e, float* sx, float* sg, float* sw,
                                         const CombArgs& prev, float* scb)
{
    static_assert(!FUSED || PER == 4, "the folded combine hands over one float4 of x per thread");
    __shared__ double red[RT_MAXW + 1], wsum[RT_MAXW], red5[3 * (RT_MAXW + 1)];
    __shared__ float wA[RT_MAXW], wP[RT_MAXW];
    const int tid = threadIdx.x, NT = blockDim.x, lane = tid & 63, wave = tid >> 6, nw = NT >> 6, d = a.d;
    TL_STAMP(a.seq, 0, 0);
    if (!FUSED && a.cbad && blockIdx.x == 0 && tid == 0) a.cbad[0] = 0;  // k_cert_select's list count
    // the input blocks b = e + g E of this workgroup, 8 threads per block counted from the last thread (the
    // last wave, while wave 0 forms the sum, bound and key): their norm weights, loaded now
    const int nb = d / 32, g = (NT - 1 - tid) >> 3, l8 = tid & 7, b = e + g * a.E, bc = min(b, nb - 1);
    const float4 nv = ((const float4*)a.pre2)[8 * bc + l8];
    const float4 fv = a.ash.q ? ((const float4*)a.fnorm)[8 * bc + l8] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    // rows staged into LDS by direct loads, one float4 per thread and round (every lane issues every load,
    // the last ones clamped to the row's end and landing in the padding of the LDS row)
    auto stage = [&](const float* src, float* dst) {
        const int n4 = d / 4;
        for (int q = 0; q * NT < n4; q++) {
            const int i = min(q * NT + tid, n4 - 1);
            __builtin_amdgcn_global_load_lds((glb_void_t)((const float4*)src + i),
                                             (lds_void_t)((float4*)dst + q * NT + wave * 64), 16, 0, 0);
        }
    };
    const int c0 = tid * PER;
    float xv[PER];
    double s2 = 0.0;
    if constexpr (FUSED) {
        // this token's x is the previous layer's combine, formed here (scb: its two LDS rows; x_new in sx
        // and in this thread's registers); its loads go out first, the router scale and W row behind them
        float4 xk;
        combine_into<1>(prev, t, sx, scb, scb + d, red5, e == 0, [&] {
            stage(a.gis, sg);
            stage(a.W + (int64_t)e * d, sw);
        }, &xk);
        xv[0] = xk.x;
        xv[1] = xk.y;
        xv[2] = xk.z;
        xv[3] = xk.w;
    } else {
        stage(a.x + (int64_t)t * d, sx);
        stage(a.gis, sg);
        stage(a.W + (int64_t)e * d, sw);
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
#pragma unroll
        for (int j = 0; j < PER; j++) xv[j] = sx[c0 + j];
    }
    // the RmsNorm scale: wave sums, then the wave totals in a fixed tree order (folded: the one barrier
    // also publishes the staged router scale and W row)
#pragma unroll
    for (int j = 0; j < PER; j++) s2 += (double)xv[j] * (double)xv[j];
    s2 = wave_sum_dpp(s2);
    if (lane == 0) red[wave] = s2;
    if constexpr (FUSED) __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    TL_STAMP(a.seq, 0, 1);
    const double S = wave_sum_dpp(lane < nw ? red[lane] : 0.0);
    const double Bs = ((double)d + 64.0) * 0x1p-52 * S;
    float mean, mhi;
    mean_ends(S, Bs, 1.0 / (double)d, &mean, &mhi);
    if (mean != mhi) {  // uniform: S is the same in every thread
        if (tid == 0) {  // (one thread: the wave routine would cost this kernel registers)
            double q = 0.0;
            for (int i = 0; i < d; i++) q += (double)sx[i] * (double)sx[i];
            red[RT_MAXW] = q;
            if (e == 0) atomicAdd(&a.flags[0], 1);
        }
        __syncthreads();
        mean = (float)(red[RT_MAXW] / (double)d);
    }
    const float rinv = rms_scale_from_mean(mean, a.eps);
    TL_STAMP(a.seq, 0, 2);
    const float sc = 1.0f / (float)__dsqrt_rn((double)d);
    float pv[PER];
    double loc = 0.0;
    float Pf = 0.0f;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        pv[j] = sw[c0 + j] * (xv[j] * rinv * sc * sg[c0 + j]);
        loc += (double)pv[j];
        Pf += fabsf(pv[j]);
    }
    const double inc = wave_incl_scan_dpp(loc);
    if (lane == 63) wsum[wave] = inc;
    __syncthreads();
    // exclusive prefix (within the double slack of the bound): the earlier waves' totals, then this wave's
    double acc = wave_sum_dpp(lane < wave ? wsum[lane] : 0.0) + (inc - loc);
    float Af = 0.0f;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        acc += (double)pv[j];
        Af += fabsf((float)acc);
    }
    Af = wave_sum_f(Af);
    Pf = wave_sum_f(Pf);
    if (lane == 0) {
        wA[wave] = Af;
        wP[wave] = Pf;
    }
    TL_STAMP(a.seq, 0, 4);
    __syncthreads();
    TL_STAMP(a.seq, 0, 5);
    // wave 0: the sum, bound and selection key; beside it, the input blocks
    if (wave == 0) {
        const double L = wave_sum_dpp(lane < nw ? wsum[lane] : 0.0);
        const float Aw = wave_sum_f(lane < nw ? wA[lane] : 0.0f);
        const float Pw = wave_sum_f(lane < nw ? wP[lane] : 0.0f);
        if (lane == 0) {
            const double As = (double)Aw * (1.0 + 0x1p-10);
            const double Ps = (double)Pw * (1.0 + 0x1p-10);
            const double B = 0x1p-24 * As * 1.001 + 0x1p-45 * Ps;
            a.Lb[(int64_t)t * a.E + e] = L;
            a.Bb[(int64_t)t * a.E + e] = B;
            a.kb[(int64_t)t * a.E + e] = sel_key(L, B, e);
        }
    }
    if (b < nb) {  // 8-lane groups: whole groups take a block or none
        const float4 xq = *(const float4*)(sx + 32 * b + 4 * l8);
        float dval;
        int sum;
        const int qw = q8_0_oct(make_float4((xq.x * rinv) * nv.x, (xq.y * rinv) * nv.y, (xq.z * rinv) * nv.z,
                                            (xq.w * rinv) * nv.w),
                                &dval, &sum);
        ((int*)(a.agu.q + (int64_t)t * a.agu.qstride))[8 * b + l8] = qw;
        if (a.agu.qh) store_qh(a.agu, t, b, l8, qw, dval);
        if (l8 == 0) {
            a.agu.d[(int64_t)t * a.agu.dstride + b] = dval;
            a.agu.s[(int64_t)t * a.agu.sstride + b] = sum;
        }
        if (a.ash.q) {
            const int qs = q8_0_oct(make_float4((xq.x * rinv) * fv.x, (xq.y * rinv) * fv.y, (xq.z * rinv) * fv.z,
                                                (xq.w * rinv) * fv.w),
                                    &dval, &sum);
            ((int*)(a.ash.q + (int64_t)t * a.ash.qstride))[8 * b + l8] = qs;
            if (a.ash.qh) store_qh(a.ash, t, b, l8, qs, dval);
            if (l8 == 0) {
                a.ash.d[(int64_t)t * a.ash.dstride + b] = dval;
                a.ash.s[(int64_t)t * a.ash.sstride + b] = sum;
            }
        }
    }
    TL_STAMP(a.seq, 0, 3);
}

// floats of one staged router row in LDS: d rounded up to whole rounds of blockDim.x float4 (the
// staging's clamped last loads land in the padding)
__host__ __device__ inline int route_row_floats(int d, int nt) { return (d / 4 + nt - 1) / nt * nt * 4; }

template <int PER, bool FUSED>
__device__ __forceinline__ void route_at(const DecArgs& a, const CombArgs& prev, float* rsm)
{
    const int t = blockIdx.x / a.E, e = blockIdx.x % a.E, dp = route_row_floats(a.d, blockDim.x);
    float* sx = rsm;
    float* sg = sx + dp;
    float* sw = sg + dp;
    float* scb = sw + dp;  // fused: the combine's two rows
    route_wg<PER, FUSED>(a, t, e, sx, sg, sw, prev, scb);
}

template <int PER>
__global__ __launch_bounds__(64 * RT_MAXW) void k_dec_route(DecArgs a)
{
    extern __shared__ __align__(16) float rsm[];  // x, router scale, W row: route_row_floats(d, NT) each
    route_at<PER, false>(a, CombArgs{}, rsm);
}

// A layer of a stack whose previous layer's combine is folded in: every (token, expert) workgroup forms
// the token's x from the previous layer's outputs (combine_into, identical in every workgroup), the
// expert-0 workgroup of each token also writes that layer's out and the new x, then the router as
// k_dec_route.  One launch fewer per layer than route + combine.
__global__ __launch_bounds__(64 * RT_MAXW) void k_dec_route_fused(CombArgs prev, DecArgs a)
{
    extern __shared__ __align__(16) float rsm[];  // x, router scale, W row, then the combine's two rows
    route_at<4, true>(a, prev, rsm);
}

// Many (token, expert) pairs (T * E > 1024, E a multiple of RT_RX): one workgroup of d / PER threads per
// token t and RT_RX consecutive experts.  The token's x row and the router scale are staged and the
// RmsNorm scale formed once for its RT_RX experts, and each expert's sum, scan and bound (route_wg's) run
// side by side; wave r finalizes expert e0 + r.  The input blocks b = g + G j (G = E / RT_RX workgroups
// per token, g this one's index) are quantized here, as route_wg quantizes b = e + E j.  (Two experts
// per workgroup measured no faster at C5: 15.6 against 15.4 us.)
constexpr int RT_RX = 4;
template <int PER>
__global__ __launch_bounds__(256) void k_dec_route_mx(DecArgs a)
{
    extern __shared__ __align__(16) float rsm[];  // x, router scale, RT_RX W rows: route_row_floats(d, NT) each
    __shared__ double red[RT_MAXW + 1], wsum[RT_RX][RT_MAXW];
    __shared__ float wA[RT_RX][RT_MAXW], wP[RT_RX][RT_MAXW];
    const int tid = threadIdx.x, NT = blockDim.x, lane = tid & 63, wave = tid >> 6, nw = NT >> 6, d = a.d;
    const int G = a.E / RT_RX, t = blockIdx.x / G, eg = blockIdx.x % G, e0 = eg * RT_RX;
    const int dp = route_row_floats(d, NT);
    float* sx = rsm;
    float* sg = sx + dp;
    float* sw = sg + dp;  // RT_RX rows of dp floats
    if (a.cbad && blockIdx.x == 0 && tid == 0) a.cbad[0] = 0;  // k_cert_select's list count
    const int nb = d / 32, g = (NT - 1 - tid) >> 3, l8 = tid & 7, b = eg + g * G, bc = min(b, nb - 1);
    const float4 nv = ((const float4*)a.pre2)[8 * bc + l8];
    const float4 fv = a.ash.q ? ((const float4*)a.fnorm)[8 * bc + l8] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    auto stage = [&](const float* src, float* dst) {
        const int n4 = d / 4;
        for (int q = 0; q * NT < n4; q++) {
            const int i = min(q * NT + tid, n4 - 1);
            __builtin_amdgcn_global_load_lds((glb_void_t)((const float4*)src + i),
                                             (lds_void_t)((float4*)dst + q * NT + wave * 64), 16, 0, 0);
        }
    };
    stage(a.x + (int64_t)t * d, sx);
    stage(a.gis, sg);
#pragma unroll
    for (int r = 0; r < RT_RX; r++) stage(a.W + (int64_t)(e0 + r) * d, sw + r * dp);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const int c0 = tid * PER;
    float xv[PER];
    double s2 = 0.0;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        xv[j] = sx[c0 + j];
        s2 += (double)xv[j] * (double)xv[j];
    }
    // the RmsNorm scale as route_wg forms it
    s2 = wave_sum_dpp(s2);
    if (lane == 0) red[wave] = s2;
    __syncthreads();
    const double S = wave_sum_dpp(lane < nw ? red[lane] : 0.0);
    float mean, mhi;
    mean_ends(S, ((double)d + 64.0) * 0x1p-52 * S, 1.0 / (double)d, &mean, &mhi);
    if (mean != mhi) {  // uniform
        if (tid == 0) {
            double q = 0.0;
            for (int i = 0; i < d; i++) q += (double)sx[i] * (double)sx[i];
            red[RT_MAXW] = q;
            if (eg == 0) atomicAdd(&a.flags[0], 1);
        }
        __syncthreads();
        mean = (float)(red[RT_MAXW] / (double)d);
    }
    const float rinv = rms_scale_from_mean(mean, a.eps);
    const float sc = 1.0f / (float)__dsqrt_rn((double)d);
    // m_i = ((x_i * rinv) * sc) * s_i, p_i = fl(W[e][i] * m_i) (route_wg's expression)
    float m[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) m[j] = xv[j] * rinv * sc * sg[c0 + j];
    double loc[RT_RX], inc[RT_RX];
    float Pf[RT_RX];
#pragma unroll
    for (int r = 0; r < RT_RX; r++) {
        loc[r] = 0.0;
        Pf[r] = 0.0f;
#pragma unroll
        for (int j = 0; j < PER; j++) {
            const float p = sw[r * dp + c0 + j] * m[j];
            loc[r] += (double)p;
            Pf[r] += fabsf(p);
        }
        inc[r] = wave_incl_scan_dpp(loc[r]);
        if (lane == 63) wsum[r][wave] = inc[r];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < RT_RX; r++) {
        // exclusive prefix: the earlier waves' totals, then this wave's
        double acc = wave_sum_dpp(lane < wave ? wsum[r][lane] : 0.0) + (inc[r] - loc[r]);
        float Af = 0.0f;
#pragma unroll
        for (int j = 0; j < PER; j++) {
            acc += (double)(sw[r * dp + c0 + j] * m[j]);
            Af += fabsf((float)acc);
        }
        Af = wave_sum_f(Af);
        const float P = wave_sum_f(Pf[r]);
        if (lane == 0) {
            wA[r][wave] = Af;
            wP[r][wave] = P;
        }
    }
    __syncthreads();
    for (int r = wave; r < RT_RX; r += nw) {  // wave r: expert e0 + r's sum, bound and selection key (route_wg's)
        const int e = e0 + r;
        const double L = wave_sum_dpp(lane < nw ? wsum[r][lane] : 0.0);
        const float Aw = wave_sum_f(lane < nw ? wA[r][lane] : 0.0f);
        const float Pw = wave_sum_f(lane < nw ? wP[r][lane] : 0.0f);
        if (lane == 0) {
            const double As = (double)Aw * (1.0 + 0x1p-10);
            const double Ps = (double)Pw * (1.0 + 0x1p-10);
            const double B = 0x1p-24 * As * 1.001 + 0x1p-45 * Ps;
            a.Lb[(int64_t)t * a.E + e] = L;
            a.Bb[(int64_t)t * a.E + e] = B;
            a.kb[(int64_t)t * a.E + e] = sel_key(L, B, e);
        }
    }
    if (b < nb) {  // 8-lane groups: whole groups take a block or none
        const float4 xq = *(const float4*)(sx + 32 * b + 4 * l8);
        float dval;
        int sum;
        const int qw = q8_0_oct(make_float4((xq.x * rinv) * nv.x, (xq.y * rinv) * nv.y, (xq.z * rinv) * nv.z,
                                            (xq.w * rinv) * nv.w),
                                &dval, &sum);
        ((int*)(a.agu.q + (int64_t)t * a.agu.qstride))[8 * b + l8] = qw;
        if (a.agu.qh) store_qh(a.agu, t, b, l8, qw, dval);
        if (l8 == 0) {
            a.agu.d[(int64_t)t * a.agu.dstride + b] = dval;
            a.agu.s[(int64_t)t * a.agu.sstride + b] = sum;
        }
        if (a.ash.q) {
            const int qs = q8_0_oct(make_float4((xq.x * rinv) * fv.x, (xq.y * rinv) * fv.y, (xq.z * rinv) * fv.z,
                                                (xq.w * rinv) * fv.w),
                                    &dval, &sum);
            ((int*)(a.ash.q + (int64_t)t * a.ash.qstride))[8 * b + l8] = qs;
            if (a.ash.qh) store_qh(a.ash, t, b, l8, qs, dval);
            if (l8 == 0) {
                a.ash.d[(int64_t)t * a.ash.dstride + b] = dval;
                a.ash.s[(int64_t)t * a.ash.sstride + b] = sum;
            }
        }
    }
}
template <int P> struct KRouteMx { static constexpr auto fn = k_dec_route_mx<P>; };

// Elements per thread: 4 (d / 4 threads) for a stack's few tokens, where the router's chain of
// reductions is the layer's latency; d / 256 (256 threads) for many tokens, where more workgroups per CU
// hide each other's barriers.  Each width is its own instantiation (its own register budget).
template <int P> struct KRoute { static constexpr auto fn = k_dec_route<P>; };
static int route_per(int T, int E, int d) { return (int64_t)T * E > 1024 ? d / 256 : 4; }
static auto route_kernel(int per)
{
    switch (per) {
    case 1: return KRoute<1>::fn;
    case 2: return KRoute<2>::fn;
    case 3: return KRoute<3>::fn;
    case 4: return KRoute<4>::fn;
    case 5: return KRoute<5>::fn;
    case 6: return KRoute<6>::fn;
    case 7: return KRoute<7>::fn;
    case 8: return KRoute<8>::fn;
    case 9: return KRoute<9>::fn;
    case 10: return KRoute<10>::fn;
    case 11: return KRoute<11>::fn;
    case 12: return KRoute<12>::fn;
    case 13: return KRoute<13>::fn;
    case 14: return KRoute<14>::fn;
    case 15: return KRoute<15>::fn;
    default: return KRoute<16>::fn;
    }
}

// ------------------------------------------------------------------------------ shared FFN workgroups
// Shared gate|up unit (in k_dec_gu): one (pair of tokens, paired row group), input from k_dec_route's
// packed Q8_0 rows.
template <int TYPE>
__device__ void shared_gu_wg(const DecArgs& a, int tile, int rgi, unsigned char* smem)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    ActL* act = (ActL*)smem;
    float* terms = (float*)(act + DROWS);
    const int t0 = tile * DROWS, cnt = min(DROWS, a.T - t0);
    ActIn ain;
    act_issue(ain, a.ash, t0, min(t0 + 1, a.T - 1), cnt, a.sgu.nb);
    __builtin_amdgcn_sched_barrier(0);  // keep the activation loads ahead of the weight loads
    WRegs<TYPE> W;
    load_w<TYPE>(a.sgu, 0, rgi, wave, lane, W);
    act_store(ain, cnt, a.sgu.nb, act);
    __syncthreads();
    const float S = rowgroup_chain<TYPE>(W, wave, a.sgu.nb, act, cnt, terms);
    if (wave < cnt) gu_epilogue(S, rgi, a.nff, t0 + wave, a.shg, a.shu, a.asd, a.gelu_tab);
}

// Shared down (in k_dec_down): one workgroup per (pair of tokens, row group).
template <int TYPE>
__device__ void shared_dn_wg(const DecArgs& a, int tile, int rgi, unsigned char* smem)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    ActL* act = (ActL*)smem;
    float* terms = (float*)(act + DROWS);
    const int t0 = tile * DROWS, cnt = min(DROWS, a.T - t0);
    ActIn ain;
    act_issue(ain, a.asd, t0, min(t0 + 1, a.T - 1), cnt, a.sdn.nb);
    __builtin_amdgcn_sched_barrier(0);  // keep the activation loads ahead of the weight loads
    WRegs<TYPE> W;
    load_w<TYPE>(a.sdn, 0, rgi, wave, lane, W);
    act_store(ain, cnt, a.sdn.nb, act);
    __syncthreads();
    const float S = rowgroup_chain<TYPE>(W, wave, a.sdn.nb, act, cnt, terms);
    const int row = rgi * 64 + lane;
    if (wave < cnt && row < a.sdn.rows) a.shout[(int64_t)(t0 + wave) * a.d + row] = S;
}

// ------------------------------------------------------------------------------ k_dec_gu
// Selection, in every expert workgroup and in the routing workgroup.  Fast path, one wave per token:
// the experts' 32-bit keys (the order-preserving bits of (float)L with the low 8 bits replaced by
// 255 - expert, so keys are distinct and ties go to the lower index) give the top-k.  The order is
// certified if each chosen expert's lower end L - B lies above the upper ends L + B of every expert
// ranked after it, compared as floats rounded outward (so a float comparison that holds implies the
// exact one); an order the key gets wrong (logits within 256 float ulps) is never certified, since
// certification compares the intervals themselves.  The router workgroup of (t, e) forms the key and
// both ends once (sel_key).  When a token is not certified, the whole workgroup takes select_exact.
// The router's logits and bounds of token t for one wave (lane + 64 q in slot q): cold reads (the router
// launch wrote them), issued at workgroup start so they travel beside the shared units' weights.
struct SelIn {
    uint4 kb[4];
};

__device__ __forceinline__ void sel_issue(const DecArgs& a, int t, SelIn& in)
{
    const int lane = threadIdx.x & 63;
    const uint4* kr = a.kb + (int64_t)t * a.E;
#pragma unroll
    for (int q = 0; q < 4; q++) in.kb[q] = kr[min(lane + 64 * q, a.E - 1)];
}

// The certified top-k of token t (one wave): k rounds of a wave maximum of the keys rank the experts;
// the order is accepted if every chosen expert's lower end lies above every later expert's upper end
// (ends rounded outward to floats); false when it cannot be (or a sum is not finite): the exact chains
// decide then.
__device__ bool wave_topk(const DecArgs& a, int t, const SelIn& in, int* s_ids, unsigned* s_klo, unsigned* s_khi)
{
    const int lane = threadIdx.x & 63, nq = (a.E + 63) / 64, k = a.k;
    unsigned key[4];
    int rank[4];
    bool fin = true;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const bool valid = q < nq && lane + 64 * q < a.E;
        key[q] = valid ? in.kb[q].x : 0u;
        if (valid && !in.kb[q].w) fin = false;
        rank[q] = 64;
    }
    for (int j = 0; j < k; j++) {
        unsigned m = max(key[0], key[1]);  // key[1] is 0 where nq == 1
        if (nq > 2) m = max(m, max(key[2], key[3]));  // uniform
        m = wave_max_u32(m);
        // the keys are distinct and nonzero: one slot of one lane matches
#pragma unroll
        for (int q = 0; q < 2; q++)
            if (key[q] == m) {
                key[q] = 0u;
                rank[q] = j;
            }
        if (nq > 2) {
#pragma unroll
            for (int q = 2; q < 4; q++)
                if (key[q] == m) {
                    key[q] = 0u;
                    rank[q] = j;
                }
        }
    }
    unsigned hun = 0u;  // the unchosen experts' highest upper end
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int ex = lane + 64 * q;
        if (rank[q] < 64) {
            s_klo[rank[q]] = in.kb[q].y;
            s_khi[rank[q]] = in.kb[q].z;
            s_ids[t * k + rank[q]] = ex;
        } else if (q < nq && ex < a.E) {
            hun = max(hun, in.kb[q].z);
        }
    }
    hun = wave_max_u32(hun);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // lane j < k: its lower end must lie above every later rank's upper end and the unchosen ones'
    // (every read issued before the first use)
    unsigned hk[PHX_MAX_USED_DEV];
#pragma unroll
    for (int r = 0; r < PHX_MAX_USED_DEV; r++) hk[r] = s_khi[r];
    const unsigned lo = s_klo[min(lane, PHX_MAX_USED_DEV - 1)];
    unsigned later = hun;
#pragma unroll
    for (int r = 0; r < PHX_MAX_USED_DEV; r++) later = (r > lane && r < k) ? max(later, hk[r]) : later;
    const bool ok = lane >= k || lo > later;
    return __all(fin && ok);
}

// LDS of the exact selection, from the start of the workgroup's union region: sL [T*E] doubles, the
// token's router input m [d] floats, the ambiguous experts' list [E] and
// four wave counts, the chosen experts' lower ends [16] and the ambiguous experts' exact keys [E]
// (doubles), and two product buffers of sel_buf_floats(NT) floats.  The host sizes the region with
// the same function.
__host__ __device__ inline size_t sel_buf_floats(int NT, int P = 1) { return (size_t)4 * P * (NT - 64) + 256; }

struct SelLds {
    size_t m, list, lo, key, buf, total;
};

__host__ __device__ inline SelLds sel_lds(int T, int E, int d, int NT, int P = 1)
{
    SelLds o;
    const size_t TE = (size_t)T * E;
    o.m = (TE * 8 + 15) & ~(size_t)15;
    o.list = o.m + (size_t)d * 4;
    o.lo = (o.list + (size_t)(E + 4) * 4 + 7) & ~(size_t)7;
    o.key = o.lo + PHX_MAX_USED_DEV * 8;
    o.buf = (o.key + (size_t)E * 8 + 15) & ~(size_t)15;
    o.total = o.buf + 2 * sel_buf_floats(NT, P) * 4;
    return o;
}

// Exact logits of ng <= 64 experts (list[0..ng-1]) for one token: the reference's float chains
// s = fl(s + fl(W[e][i] * m_i)), i = 0..d-1 in order, from s = 0 (src/GemmaCpu.cs:389-395).  Waves
// 1..NWV-1 form the products of one segment of seg = 4 * segq elements of every chain per step (one
// float4 each, its W loads issued PD steps ahead) into one of two LDS buffers; lane j of wave 0 adds
// chain j's previous segment from the other buffer in index order, its LDS reads eight float4 ahead of
// the adds.  One barrier per step.  The chains' sums go to out[list[j]] as doubles.
constexpr int SEL_PD = 4;

__device__ void exact_chains(const float* W, int d, const float* sm, const int* list, int ng, float* sbuf,
                             size_t bufn, double* out)
{
    ng = __builtin_amdgcn_readfirstlane(ng);  // uniform (an LDS count): scalar loop control
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), NPT = blockDim.x - 64;
    const int sq = NPT / ng, segq = min(sq >= 16 ? sq & ~15 : sq, d / 4), seg = 4 * segq, stride = seg + 4;
    const int nseg = (d + seg - 1) / seg;
    // producer q = tid - 64: chain jq, float4 slot oq of the segment (idle when jq >= ng).  Every thread
    // issues the loads (wave 0 and idle producers at clamped, valid addresses), so no branch separates
    // a load from its use and the loads of later steps stay in flight.
    const int q = tid >= 64 ? tid - 64 : tid, jq = q / segq, oq = q - jq * segq;
    const bool prod = wave > 0 && jq < ng;
    const float4* wrow = (const float4*)(W + (int64_t)list[min(jq, ng - 1)] * d);
    const int n4 = d / 4;
    float4 r[SEL_PD];
#pragma unroll
    for (int k = 0; k < SEL_PD; k++) {
        r[k] = wrow[min(k * segq + oq, n4 - 1)];
        __builtin_amdgcn_sched_barrier(0);  // in step order, as the loop issues them: a step waits on its own
    }
    float s = 0.0f;
    for (int s0 = 0; s0 <= nseg; s0 += SEL_PD) {  // steps 0..nseg, padded to whole groups of PD
#pragma unroll
        for (int k = 0; k < SEL_PD; k++) {
            const int st = s0 + k;
            const int i4 = st * segq + oq;
            if (prod && st < nseg && i4 < n4) {
                const float4 m = ((const float4*)sm)[i4];
                float4 p;
                p.x = r[k].x * m.x;
                p.y = r[k].y * m.y;
                p.z = r[k].z * m.z;
                p.w = r[k].w * m.w;
                *(float4*)(sbuf + (st & 1) * bufn + jq * stride + 4 * oq) = p;
            }
            r[k] = wrow[min((st + SEL_PD) * segq + oq, n4 - 1)];  // the step PD ahead (clamped)
            if (wave == 0 && st >= 1 && st <= nseg && tid < ng) {
                const int sp = st - 1, c4 = min(segq, n4 - sp * segq);
                const float4* b4 = (const float4*)(sbuf + (sp & 1) * bufn + tid * stride);
                // batches of sixteen float4: the batch's reads go out together and the adds of its first
                // float4 wait for one LDS round trip, the rest arrive while the earlier ones are added
                const int c16 = c4 & ~15;
                for (int c = 0; c < c16; c += 16) {
                    float4 v[16];
#pragma unroll
                    for (int u = 0; u < 16; u++) v[u] = b4[c + u];
#pragma unroll
                    for (int u = 0; u < 16; u++) {
                        s += v[u].x;
                        s += v[u].y;
                        s += v[u].z;
                        s += v[u].w;
                    }
                }
                for (int c = c16; c < c4; c++) {
                    const float4 t = b4[c];
                    s += t.x;
                    s += t.y;
                    s += t.z;
                    s += t.w;
                }
            }
            __syncthreads();
        }
    }
    if (wave == 0 && tid < ng) out[list[tid]] = (double)s;
    __syncthreads();
}

// The fallback kernel's chains (exact_chains' arithmetic and order): each producer forms CF_P float4 of
// products per step, so a chain's segment per step is CF_P times longer (fewer barriers), the W loads
// for the next step issued right after the current step's products; the adding lane reads its segment
// with explicit LDS reads, 32 float4 per round trip.
constexpr int CF_P = 2;
__device__ void exact_chains_wide(const float* W, int d, const float* sm, const int* list, int ng, float* sbuf,
                                  size_t bufn, double* out)
{
    ng = __builtin_amdgcn_readfirstlane(ng);
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), NPT = blockDim.x - 64;
    const int sq = CF_P * NPT / ng, segq = min(sq >= 32 ? sq & ~31 : sq, d / 4), seg = 4 * segq, stride = seg + 4;
    const int nseg = (d + seg - 1) / seg, n4 = d / 4;
    const float4* sm4 = (const float4*)sm;
    // producer q = tid - 64: slots q + p NPT of the step (chain j, float4 o), idle past ng * segq
    const int q = tid >= 64 ? tid - 64 : 0;
    int jq[CF_P], oq[CF_P];
    bool act[CF_P];
    const float4* wr[CF_P];
    float4 r[CF_P];
#pragma unroll
    for (int p = 0; p < CF_P; p++) {
        const int sl = q + p * NPT;
        jq[p] = sl / segq;
        oq[p] = sl - jq[p] * segq;
        act[p] = wave > 0 && jq[p] < ng;
        wr[p] = (const float4*)(W + (int64_t)list[min(jq[p], ng - 1)] * d);
        r[p] = wr[p][min(oq[p], n4 - 1)];
    }
    float s = 0.0f;
    const uint32_t abase = (uint32_t)(uintptr_t)(lds_void_t)(sbuf + tid * stride);
    for (int st = 0; st <= nseg; st++) {
        if (st < nseg) {
#pragma unroll
            for (int p = 0; p < CF_P; p++) {
                const int i4 = st * segq + oq[p];
                if (act[p] && i4 < n4) {
                    const float4 m = sm4[i4];
                    float4 v;
                    v.x = r[p].x * m.x;
                    v.y = r[p].y * m.y;
                    v.z = r[p].z * m.z;
                    v.w = r[p].w * m.w;
                    *(float4*)(sbuf + (st & 1) * bufn + jq[p] * stride + 4 * oq[p]) = v;
                }
            }
#pragma unroll
            for (int p = 0; p < CF_P; p++) r[p] = wr[p][min((st + 1) * segq + oq[p], n4 - 1)];  // the next step's
        }
        if (wave == 0 && st >= 1 && tid < ng) {
            const int sp = st - 1, c4 = min(segq, n4 - sp * segq), c32 = c4 & ~31;
            const uint32_t a0 = abase + (uint32_t)((sp & 1) * bufn * 4);
            for (int c = 0; c < c32; c += 32) {
                u32x4 v[32];
                static_for<32>([&](auto U) { v[decltype(U)::value] = ds_r128<16 * decltype(U)::value>(a0 + 16 * c); });
                static_for<32>([&](auto U) {
                    constexpr int u = decltype(U)::value;
                    // two waits per batch (a wait per float4 would cost an issue slot per four adds): at
                    // most 15 LDS reads are outstanding (the counter's width), so the first 17 have landed
                    // once 15 remain; the rest long before the first 17 are added
                    if constexpr (u == 0) asm volatile("s_waitcnt lgkmcnt(15)" ::: "memory");
                    if constexpr (u == 17) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                    tie(v[u]);
                    s += __uint_as_float(v[u].x);
                    s += __uint_as_float(v[u].y);
                    s += __uint_as_float(v[u].z);
                    s += __uint_as_float(v[u].w);
                });
            }
            const float4* b4 = (const float4*)(sbuf + (sp & 1) * bufn + tid * stride);
            for (int c = c32; c < c4; c++) {
                const float4 t = b4[c];
                s += t.x;
                s += t.y;
                s += t.z;
                s += t.w;
            }
        }
        __syncthreads();
    }
    if (wave == 0 && tid < ng) out[list[tid]] = (double)s;
    __syncthreads();
}

// Exact selection for the tokens marked in s_bad (rare): the experts that can reach the chosen ones
// (the ambiguous ones) are recomputed as the reference's float chains (src/GemmaCpu.cs:389-395) and
// ranked exactly by the strict '>' scan of GemmaCpu.cs:400-405 (ties to the lower index; a NaN
// logit is taken once every lower-index expert is).  Every other expert's upper end lies below every
// chosen expert's lower end, so the top-k lies among the ambiguous ones, unless a chain ends
// non-finite: then every expert of the token is recomputed and ranked.  un: the LDS of sel_lds; sL (at un) ends holding the logits
// the routing reports for those tokens.
// PIPE: the fallback kernel's variant (the rms scales the many-token router formed, when given)
template <bool PIPE = false>
__device__ void select_exact(const DecArgs& a, unsigned char* un, int* s_ids, const int* s_bad, double* red,
                             bool count)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, NT = blockDim.x;
    const SelLds lds = sel_lds(a.T, a.E, a.d, NT, PIPE ? CF_P : 1);
    double* sL = (double*)un;
    float* sm = (float*)(un + lds.m);
    int* slist = (int*)(un + lds.list);
    int* swc = slist + a.E;
    double* slo = (double*)(un + lds.lo);
    double* skey = (double*)(un + lds.key);
    float* sbuf = (float*)(un + lds.buf);
    const float sc = 1.0f / (float)__dsqrt_rn((double)a.d);
    const int E = a.E, k = a.k, nwe = (E + 63) / 64;
    // elements per thread per load round of the token's row (the decode kernel's variant keeps one: its
    // registers are the roofline kernel's)
    constexpr int RB = PIPE ? 8 : 1;
    for (int tt = 0; tt < a.T; tt++) {
        if (!s_bad[tt]) continue;  // uniform: an LDS value read after a barrier
        if (count && tid == 0) atomicAdd(&a.flags[1], 1);
        const float* xr = a.x + (int64_t)tt * a.d;
        const double* Lr = a.Lb + (int64_t)tt * E;
        const double* Br = a.Bb + (int64_t)tt * E;
        // the bounds (thread b: expert b) and the chosen experts' lower ends, loaded beside x
        double lb = 0.0, bb = 0.0;
        if (tid < E) {
            lb = Lr[tid];
            bb = Br[tid];
        }
        if (tid < k) {
            const int ex = s_ids[tt * k + tid];
            slo[tid] = Lr[ex] - Br[ex];
        }
        float rinv_t;
        if (PIPE && a.xscale) {  // the router's (the same certified mean and expression)
            rinv_t = a.xscale[tt];
        } else {
            double s = 0.0;
            for (int i0 = tid; i0 < a.d; i0 += RB * NT) {  // RB loads per round, then the terms in order
                float xv[RB];
#pragma unroll
                for (int u = 0; u < RB; u++) xv[u] = xr[min(i0 + u * NT, a.d - 1)];
#pragma unroll
                for (int u = 0; u < RB; u++)
                    if (i0 + u * NT < a.d) s += (double)xv[u] * (double)xv[u];
            }
            rinv_t = rms_scale_from_mean(wg_mean_sq<true, PIPE>(s, xr, a.d, red, nullptr), a.eps);
        }
        for (int i0 = tid; i0 < a.d; i0 += RB * NT) {  // RB elements per round: every load, then the stores
            float xv[RB], gv[RB];
#pragma unroll
            for (int u = 0; u < RB; u++) {
                const int i = min(i0 + u * NT, a.d - 1);
                xv[u] = xr[i];
                gv[u] = a.gis[i];
            }
#pragma unroll
            for (int u = 0; u < RB; u++)
                if (i0 + u * NT < a.d) sm[i0 + u * NT] = ((xv[u] * rinv_t) * sc) * gv[u];
        }
        const bool nonfinite = __syncthreads_or(tid < E && !(isfinite(lb) && isfinite(bb)));  // publishes sm, slo
        // the lowest lower end among the fast path's chosen experts: an expert whose upper end does not
        // reach it ranks below every chosen one in exact arithmetic too
        double minlo = INFINITY;
        for (int j = 0; j < k; j++) minlo = fmin(minlo, slo[j]);
        int na = 0;
        for (int all = nonfinite; all < 2; all++) {
            // the ambiguous experts in index order: one per lane of waves 0..nwe-1
            bool amb = false;
            uint64_t m = 0;
            if (wave < nwe) {
                if (tid < E) {
                    amb = all || !(lb + bb < minlo);
                    sL[tt * E + tid] = lb;
                }
                m = __ballot(amb);
                if (lane == 0) swc[wave] = __popcll(m);
            }
            __syncthreads();
            int off = 0;
            na = 0;
            for (int w = 0; w < nwe; w++) {
                const int c = swc[w];
                if (w < wave) off += c;
                na += c;
            }
            if (amb) slist[off + __popcll(m & ((1ull << lane) - 1))] = tid;
            __syncthreads();
            for (int g0 = 0; g0 < na; g0 += 64)
                if constexpr (PIPE)
                    exact_chains_wide(a.W, a.d, sm, slist + g0, min(64, na - g0), sbuf, sel_buf_floats(NT, CF_P),
                                      sL + tt * E);
                else
                    exact_chains(a.W, a.d, sm, slist + g0, min(64, na - g0), sbuf, sel_buf_floats(NT), sL + tt * E);
            if (all) break;
            // a non-finite chain (overflow) voids the bounds' argument: recompute every expert
            const bool nfc = tid < na && !isfinite(sL[tt * E + slist[tid]]);
            if (!__syncthreads_or(nfc)) break;
        }
        // exact ranks among the ambiguous experts (slist holds them in index order, so list position
        // order is expert order).  A non-NaN expert's rank r among the non-NaN ones is the count of
        // those that beat it.  A NaN logit appears only with every expert in the list, and the
        // reference's scan (see scan_start) takes a NaN expert as soon as every lower-index expert is
        // taken: right after the last-ranked non-NaN expert below it (rank P, -1 when there is none),
        // behind the NaN experts below it.  So a NaN expert's position is P + 1 + (NaN experts below
        // it) and a non-NaN expert's is r + (NaN experts whose P lies below r).
        if (tid < na) skey[tid] = sL[tt * E + slist[tid]];
        __syncthreads();
        const double my = tid < na ? skey[tid] : 0.0;
        const bool my_nan = tid < na && my != my;
        int r = 0;
        if (tid < na && !my_nan)
            for (int c = 0; c < na; c++) {
                const double o = skey[c];
                r += o == o && sel_beats(o, c, my, tid);
            }
        if (__syncthreads_or(my_nan)) {  // uniform; sbuf is free once the chains are done
            int* srank = (int*)sbuf;     // [na] ranks of the non-NaN experts
            int* sprev = srank + E;      // [na] P of the NaN experts, INT_MAX for the others
            if (tid < na) srank[tid] = r;
            __syncthreads();
            int P = -1, below = 0;
            if (my_nan)
                for (int c = 0; c < tid; c++) {
                    const double o = skey[c];
                    if (o != o) below++;
                    else P = max(P, srank[c]);
                }
            if (tid < na) sprev[tid] = my_nan ? P : INT_MAX;
            __syncthreads();
            if (my_nan) {
                r = P + 1 + below;
            } else if (tid < na) {
                int ahead = 0;
                for (int c = 0; c < na; c++) ahead += sprev[c] < r;
                r += ahead;
            }
        }
        if (tid < na && r < k) s_ids[tt * k + r] = slist[tid];
        __syncthreads();
    }
}

// Expert lists (ascending assignment order within each expert, the lists of KernelsMoe.Bucket,
// src/KernelsMoe.cs:281-330) and tiles of <= DROWS assignments, from s_ids into LDS.  The
// workgroup has at least max(E, T * k) threads.
__device__ void build_tiles(const DecArgs& a, const int* s_ids, int* s_cnt, int* s_off, int* s_tb, int* s_perm,
                            DecTile* s_tiles, int* s_nt, int* wtot)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, NT = blockDim.x;
    const int n = a.T * a.k;
    for (int x = tid; x <= a.E; x += NT) s_cnt[x] = 0;
    __syncthreads();
    int my_e = 0, my_rank = 0;
    if (tid < n) {
        my_e = clamp_id(s_ids[tid], a.E);
        for (int b = 0; b < tid; b++) my_rank += clamp_id(s_ids[b], a.E) == my_e;
        atomicAdd(&s_cnt[my_e], 1);
    }
    __syncthreads();
    // exclusive scans of the counts and of the tile counts (one expert per thread)
    {
        const int c = tid < a.E ? s_cnt[tid] : 0;
        const int tcount = (c + DROWS - 1) / DROWS;
        const int v1 = wave_incl_scan_i(c), v2 = wave_incl_scan_i(tcount);
        if (lane == 63) {
            wtot[wave] = v1;
            wtot[16 + wave] = v2;
        }
        __syncthreads();
        int b1 = 0, b2 = 0;
        for (int w = 0; w < wave; w++) {
            b1 += wtot[w];
            b2 += wtot[16 + w];
        }
        if (tid < a.E) {
            s_off[tid] = b1 + v1 - c;
            s_tb[tid] = b2 + v2 - tcount;
        }
        if (tid == 0) {
            int t1 = 0, t2 = 0;
            for (int w = 0; w < NT / 64; w++) {
                t1 += wtot[w];
                t2 += wtot[16 + w];
            }
            s_off[a.E] = t1;
            *s_nt = t2;
        }
        __syncthreads();
    }
    if (tid < n) s_perm[s_off[my_e] + my_rank] = tid;
    __syncthreads();
    if (tid < a.E) {
        const int c = s_cnt[tid], base = s_tb[tid];
        for (int q = 0; q * DROWS < c; q++) {
            const int st0 = s_off[tid] + q * DROWS, m = min(DROWS, c - q * DROWS);
            s_tiles[base + q] = DecTile{tid, m, {s_perm[st0], m > 1 ? s_perm[st0 + 1] : 0}};
        }
    }
    __syncthreads();
}

// Routing outputs (workgroup 0): ids, logits, weights (src/GemmaCpu.cs:406-407,417: p_j = exp in
// double, sum in double, w_j = (float)(p_j / sum) * down_scale), offsets, lists and the tile list of
// k_dec_down.  Lr(t, e) gives the logit the routing used.
template <class LF>
__device__ void write_routing(const DecArgs& a, LF Lr, const int* s_ids, const int* s_off, const int* s_perm,
                              const DecTile* s_tiles, int ntiles)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, NT = blockDim.x;
    const int TE = a.T * a.E, n = a.T * a.k;
    for (int i = tid; i < TE; i += NT) a.logits[i] = (float)Lr(i / a.E, i % a.E);
    for (int x = tid; x <= a.E; x += NT) a.offsets[x] = s_off[x];
    for (int i = tid; i < n; i += NT) a.perm[i] = s_perm[i];
    for (int q = tid; q < a.max_tiles; q += NT) a.tiles[q] = q < ntiles ? s_tiles[q] : DecTile{-1, 0, {0, 0}};
    for (int tt = wave; tt < a.T; tt += NT / 64) {
        const int j = lane;
        const bool act = j < a.k;
        const int id = act ? s_ids[tt * a.k + j] : 0;
        const float selj = act ? (float)Lr(tt, id) : 0.0f;
        const float sel0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(selj), 0));
        // p_0 = exp(0) = 1 exactly, so the CPU's in-place rule uses 1 for every later term
        const float top = (a.rule == 1 && j > 0) ? 1.0f : sel0;
        const float pj = act ? (float)exp((double)(selj - top)) : 0.0f;
        double sum = 0.0;
        for (int q = 0; q < a.k; q++)  // in rank order
            sum += (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(pj), q));
        if (act) {
            a.ids[(int64_t)tt * a.k + j] = id;
            a.w[(int64_t)tt * a.k + j] = (float)((double)pj / sum) * a.ds[id];
        }
    }
}

// One token's routing outputs from one wave: its logits (Lr: the exact chains' values where the
// selection ran them, the certified sums elsewhere), ids and weights (src/GemmaCpu.cs:406-407,417, as
// write_routing).
__device__ void token_routing_out(const DecArgs& a, int t, const double* Lr, const int* s_ids)
{
    const int lane = threadIdx.x & 63;
    for (int e = lane; e < a.E; e += 64) a.logits[(int64_t)t * a.E + e] = (float)Lr[e];
    const int j = lane;
    const bool act = j < a.k;
    const int id = act ? s_ids[j] : 0;
    const float selj = act ? (float)Lr[id] : 0.0f;
    const float sel0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(selj), 0));
    const float top = (a.rule == 1 && j > 0) ? 1.0f : sel0;
    const float pj = act ? (float)exp((double)(selj - top)) : 0.0f;
    double sum = 0.0;
    for (int q = 0; q < a.k; q++)  // in rank order
        sum += (double)__int_as_float(__builtin_amdgcn_readlane(__float_as_int(pj), q));
    if (act) {
        a.ids[(int64_t)t * a.k + j] = id;
        a.w[(int64_t)t * a.k + j] = (float)((double)pj / sum) * a.ds[id];
    }
}

// The token's own view of the certified sums (one token)
__device__ __forceinline__ DecArgs token_view(const DecArgs& a, int t)
{
    DecArgs b = a;
    b.T = 1;
    b.x = a.x + (int64_t)t * a.d;
    b.xscale = a.xscale ? a.xscale + t : nullptr;
    b.Lb = a.Lb + (int64_t)t * a.E;
    b.Bb = a.Bb + (int64_t)t * a.E;
    b.kb = a.kb + (int64_t)t * a.E;
    return b;
}

// The general path's selection from the certified routers (k_dec_route's or k_router_mm's sums and
// bounds), one wave per token: the fast path of wave_topk and the token's ids, weights and logits; a
// token whose order the bounds leave open is marked in bad[] for k_cert_fallback.
constexpr int CS_TPW = 4;  // tokens (waves) per workgroup
__global__ __launch_bounds__(64 * CS_TPW) void k_cert_select(DecArgs a)
{
    __shared__ int s_ids[CS_TPW][PHX_MAX_USED_DEV];
    __shared__ unsigned s_kb[CS_TPW][2 * PHX_MAX_USED_DEV];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int t = blockIdx.x * CS_TPW + wave;
    if (t >= a.T) return;  // wave-uniform; no workgroup barrier follows
    const DecArgs b = token_view(a, t);
    SelIn in;
    sel_issue(b, 0, in);
    const bool cert = wave_topk(b, 0, in, s_ids[wave], s_kb[wave], s_kb[wave] + PHX_MAX_USED_DEV);
    if (cert) {
        token_routing_out(a, t, b.Lb, s_ids[wave]);
    } else {
        if (lane < a.k) a.ids[(int64_t)t * a.k + lane] = s_ids[wave][lane];  // provisional: their lower ends
        if (lane == 0) a.cbad[1 + atomicAdd(&a.cbad[0], 1)] = t;  // (the router cleared the count)
    }
}

// The tokens k_cert_select listed: the exact selection (select_exact, counted as router fallbacks)
// with a workgroup of CF_NT threads per token, so that each chain's segment per step is long; workgroup
// g takes the listed tokens g, g + G, ... (G workgroups).
constexpr int CF_NT = 512;
__global__ __launch_bounds__(CF_NT) void k_cert_fallback(DecArgs a)
{
    extern __shared__ __align__(16) unsigned char csm[];  // sel_lds(1, E, d, CF_NT)
    __shared__ int s_ids[PHX_MAX_USED_DEV];
    __shared__ double red[CF_NT / 64 + 1];
    __shared__ int s_one;
    const int tid = threadIdx.x, wave = tid >> 6, G = gridDim.x;
    if (tid == 0) s_one = 1;
    const int n = a.cbad[0];
    for (int q = blockIdx.x; q < n; q += G) {  // uniform
        const int tt = a.cbad[1 + q];
        const DecArgs b = token_view(a, tt);
        if (tid < a.k) s_ids[tid] = a.ids[(int64_t)tt * a.k + tid];  // k_cert_select's provisional top-k
        __syncthreads();
        select_exact<true>(b, csm, s_ids, &s_one, red, true);
        if (wave == 0) token_routing_out(a, tt, (const double*)csm, s_ids);
        __syncthreads();
    }
}

// Few tokens (at most two workgroups per compute unit): one workgroup of CF_NT threads per token, the
// fast path in wave 0 and, for a token the bounds leave open, the exact selection in the same launch.
__global__ __launch_bounds__(CF_NT) void k_cert_select_one(DecArgs a)
{
    extern __shared__ __align__(16) unsigned char csm[];  // sel_lds(1, E, d, CF_NT, CF_P)
    __shared__ int s_ids[PHX_MAX_USED_DEV];
    __shared__ unsigned s_kb[2 * PHX_MAX_USED_DEV];
    __shared__ double red[CF_NT / 64 + 1];
    __shared__ int s_bad;
    const int t = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const DecArgs b = token_view(a, t);
    if (wave == 0) {
        SelIn in;
        sel_issue(b, 0, in);
        const bool cert = wave_topk(b, 0, in, s_ids, s_kb, s_kb + PHX_MAX_USED_DEV);
        if (lane == 0) s_bad = !cert;
    }
    __syncthreads();
    const bool exact = s_bad != 0;  // uniform
    if (exact) select_exact<true>(b, csm, s_ids, &s_bad, red, true);
    if (wave == 0) token_routing_out(a, t, exact ? (const double*)csm : b.Lb, s_ids);
}

// ------------------------------------------------------------------------------ k_router_mm
// The certified router for many tokens, where a workgroup per (token, expert) no longer pays: the
// logits of a tile of TM tokens x TN experts as fp32 matrix-core sums, with the bound k_cert_select
// certifies the top-k order from (the decode router's L, B, keys; the reference chain is
// src/GemmaCpu.cs:389-395, its input m_i = ((x_i * rinv) * sc) * s_i, :388-389, rinv the row's rms scale,
// CpuRef.cs:183-191).
//
// Split over the reduction: wave w of the RM_NW waves sums the chunks [c0, c0 + cnt) of 16 elements
// of every logit of the tile (router_range; v_mfma_f32_16x16x4_f32; lane group g of a 16 x 16 product
// holds the elements 4 g .. 4 g + 3 of the chunk, so the four products of a chunk cover it whole), and
// adds |C_j|, its accumulator after each chunk j, to a sum.  Each wave streams its own operands through
// an LDS ring of RING chunks (one direct global -> LDS load per 16 rows: x and the prescaled router
// rows), so no barrier is needed inside the loop.
//
// The bound.  With p_i = fl(m_i w_i), S_k = sum_{i <= k} p_i and u = 2^-24, the reference's chain
// ends within 1.004 u sum_k |S_k| of S_n (n <= 65536).  The matrix cores sum a_i w'_i with a_i = x_i
// and w'_i = fl(s_i w_i) (the rows prescaled at upload), and the row's factor f = rinv / sqrt(d) (exact
// in double) scales the sums: p_i carries four roundings (three in m_i, one in the product) and
// f a_i w'_i one, so f a_i w'_i stands in for p_i within 5u |f a_i w'_i|.  Range r
// (n_r elements, exact prefix O_r at its start) gives sum_{k in r} |S_k| <= n_r |O_r| + 16 sum_j |Q_rj|
// + 15 sum_r |p| (Q_rj the range's own prefix at the end of chunk j: within a chunk each prefix differs
// from the chunk end's by at most the chunk's |p|).  A 4-deep fp32 product rounds at most five times,
// each to nearest, so the matrix cores' sum differs from the exact one of the exact products by at
// most 5 u (|C_in| + sum |a b|) per instruction, summed: 20 u (sum_j |C_j| + sum |a w|) over a range
// (every instruction's C_in lies within the chunk's |a w| of the chunk's start).  Together, with the
// second-order terms (the n_r-fold ranges' errors, the float sums of |C_j| and of the squares) inside
// the 1.03 factor and the coefficient of the last sum:
//   |S_ref - L| <= 1.03 u f (sum_r n_r |O_r| + 36 sum_rj |C_rj| + 44 sum_r |a_r| |w_r|)
//                  + 2^-50 f sum_r |C_r| + 2^-90 n (1 + f),
// sum |a w'| bounded per range by Cauchy-Schwarz (|a_r|^2 the range's double sum of squares of x, |w'_r|^2
// formed at upload and rounded up), O_r from the waves' unscaled totals, L = f times their
// double sum; the last terms cover L's double roundings and products or sums the matrix cores flush
// below 2^-126.  A bound of 2^100 or more (or a non-finite one) is made infinite: the token then takes
// the exact chains for every expert, as for a non-finite logit.  The rows' rms scales come from the
// waves' double sums of squares, certified as the prologue certifies them, so this kernel needs no
// input from the prologue.
constexpr int RM_NW = kRouterRanges;
template <int TM16, int TN16>
struct RmLds {
    static constexpr int TM = 16 * TM16, TN = 16 * TN16;
    static constexpr int SLOT = (TM + TN) * 64;  // [TM x rows][TN W' rows] of 16 floats
    static constexpr int DMA = TM16 + TN16;      // direct loads per chunk and wave
    // ring depth: the chunks a wave keeps in flight (deeper rings, 160 KB of LDS at 32 x 32 and 128 KB at
    // 16 x 16, measured no faster: C3 30.3 -> 27.7 us but the side stream's prologue then finds no room
    // beside it and the layer got slower; C4 18.2 -> 18.8 us)
    static constexpr int RING = 4;
    static constexpr int RINGS = RM_NW * RING * SLOT;
    // per wave: C, sum |C_j| (floats), |w'|^2 (floats), the tokens' sums of squares (doubles); the tokens' scales
    static constexpr int FIN = RM_NW * (2 * TM * TN + TN) * 4 + RM_NW * TM * 8 + TM * 4;
    static constexpr int BYTES = RINGS > FIN ? RINGS : FIN;
};
typedef float mf4v __attribute__((ext_vector_type(4)));

struct RmArgs {
    int T, d, E;
    float eps;
    const float *x, *W, *Wn;   // x [T][d], W [E][d] the prescaled router rows, Wn [E][RM_NW] their range norms^2
    float* xscale;             // [T] out: the rows' rms scales (the exact selection's)
    double *Lb, *Bb;
    uint4* kb;
    int* cbad;   // the selection's list of uncertified tokens: its count is cleared here
    int* flags;  // [0] the rows whose certified mean fell back to the sequential sum
};

// (a device function: the direct loads' builtin inside a kernel's own lambdas leaves the host side
// without the kernel's launch stub)
template <int TM16, int TN16>
__device__ __forceinline__ void router_mm_tile(const RmArgs& a, unsigned char* rmsm)
{
    using RG = RmLds<TM16, TN16>;
    constexpr int TM = RG::TM, TN = RG::TN;
    const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, r = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int t0 = blockIdx.x * TM, e0 = blockIdx.y * TN;
    int c0, cnt;
    router_range(a.d, wave, &c0, &cnt);
    constexpr int RM_RING = RG::RING;
    unsigned char* ring = rmsm + wave * (RM_RING * RG::SLOT);
    const uint32_t ring0 = (uint32_t)(uintptr_t)(lds_void_t)ring;
    if (tid == 0 && blockIdx.x == 0 && blockIdx.y == 0) a.cbad[0] = 0;

    // direct-load sources: row 16 s + lane / 4 of the tile, 16 bytes (lane % 4) of the chunk; rows past
    // the end load the last one (never stored)
    uint32_t vx[TM16], vw[TN16];
#pragma unroll
    for (int s = 0; s < TM16; s++) vx[s] = (uint32_t)((min(t0 + 16 * s + (lane >> 2), a.T - 1) * a.d + 4 * (lane & 3)) * 4);
#pragma unroll
    for (int s = 0; s < TN16; s++) vw[s] = (uint32_t)((min(e0 + 16 * s + (lane >> 2), a.E - 1) * a.d + 4 * (lane & 3)) * 4);
    const __amdgpu_buffer_rsrc_t r_x = buf_rsrc(a.x), r_w = buf_rsrc(a.W);
#define RM_LOAD(rsrc, off, voff, soff) \
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t)(ring + (off)), 16, voff, soff, 0, 0)
    auto issue = [&](auto SC, int j) {  // chunk j of the wave's range into slot S (past the end: the last again)
        constexpr int S = decltype(SC)::value;
        const uint32_t so = (uint32_t)((c0 + min(j, cnt - 1)) * 64);
#pragma unroll
        for (int s = 0; s < TM16; s++) RM_LOAD(r_x, S * RG::SLOT + 1024 * s, vx[s], so);
#pragma unroll
        for (int s = 0; s < TN16; s++) RM_LOAD(r_w, S * RG::SLOT + TM * 64 + 1024 * s, vw[s], so);
    };
#undef RM_LOAD

    mf4v acc[TM16][TN16], sab[TM16][TN16];
    double s2[TM16];  // the rows' sums of squares (this lane's elements)
#pragma unroll
    for (int i = 0; i < TM16; i++) {
        s2[i] = 0.0;
#pragma unroll
        for (int j = 0; j < TN16; j++) acc[i][j] = sab[i][j] = mf4v{0.0f, 0.0f, 0.0f, 0.0f};
    }
    // the lane's LDS read addresses: x row 16 i + r, W' row 16 j + r, 16 bytes g
    const uint32_t a_x = ring0 + r * 64 + 16 * g, a_w = a_x + TM * 64;

    auto step = [&](auto SC, int j) {
        constexpr int S = decltype(SC)::value;
        __builtin_amdgcn_s_waitcnt(vm_wait(RG::DMA * (RM_RING - 1)));  // chunk j landed (the later ones may not)
        u32x4 X[TM16], Wv[TN16];
        static_for<TM16>([&](auto I) { X[I] = ds_r128<S * RG::SLOT + 1024 * decltype(I)::value>(a_x); });
        static_for<TN16>([&](auto J) { Wv[J] = ds_r128<S * RG::SLOT + 1024 * decltype(J)::value>(a_w); });
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int i = 0; i < TM16; i++) tie(X[i]);
#pragma unroll
        for (int jj = 0; jj < TN16; jj++) tie(Wv[jj]);
        // x as it is (the row's scale rinv / sqrt(d) is applied to the sums), W' prescaled at upload
        float m[TM16][4], w[TN16][4];
#pragma unroll
        for (int i = 0; i < TM16; i++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                m[i][q] = __uint_as_float(X[i][q]);
                s2[i] = fma((double)m[i][q], (double)m[i][q], s2[i]);  // x^2 exact in double: one rounding either way
            }
#pragma unroll
        for (int jj = 0; jj < TN16; jj++)
#pragma unroll
            for (int q = 0; q < 4; q++) w[jj][q] = __uint_as_float(Wv[jj][q]);
#pragma unroll
        for (int q = 0; q < 4; q++)
#pragma unroll
            for (int i = 0; i < TM16; i++)
#pragma unroll
                for (int jj = 0; jj < TN16; jj++)
                    acc[i][jj] = __builtin_amdgcn_mfma_f32_16x16x4f32(m[i][q], w[jj][q], acc[i][jj], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < TM16; i++)
#pragma unroll
            for (int jj = 0; jj < TN16; jj++)
#pragma unroll
                for (int v = 0; v < 4; v++) sab[i][jj][v] += fabsf(acc[i][jj][v]);
    };
    // chunk j + RM_RING - 1 goes into the slot chunk j - 1 left (its reads ended in step j - 1) before
    // step j
    static_for<RM_RING - 1>([&](auto S) { issue(S, decltype(S)::value); });
    for (int j = 0; j < cnt; j += RM_RING) {
        static_for<RM_RING>([&](auto S) {
            constexpr int sl = decltype(S)::value;
            if (j + sl < cnt) {
                issue(ic<(sl + RM_RING - 1) % RM_RING>{}, j + sl + RM_RING - 1);
                step(S, j + sl);
            }
        });
    }
    __builtin_amdgcn_s_waitcnt(vm_wait(0));  // the clamped reloads past the end (into this wave's ring)

    // the squares' sums over the four lane groups (each lane: its group's elements of row r)
#pragma unroll
    for (int i = 0; i < TM16; i++) {
        s2[i] += __shfl_xor(s2[i], 16);
        s2[i] += __shfl_xor(s2[i], 32);
    }
    __syncthreads();  // every wave is done with its ring
    float* fC = (float*)rmsm;          // [wave][TM][TN] the range's sum
    float* fS = fC + RM_NW * TM * TN;  // [wave][TM][TN] its sum of |C_j|
    float* fW = fS + RM_NW * TM * TN;  // [wave][TN] |w'|^2 over the range (from upload)
    double* fQ = (double*)(fW + RM_NW * TN);  // [wave][TM] the rows' sums of squares over the range
    float* fR = (float*)(fQ + RM_NW * TM);    // [TM] the rows' rms scales
#pragma unroll
    for (int i = 0; i < TM16; i++)
#pragma unroll
        for (int jj = 0; jj < TN16; jj++)
#pragma unroll
            for (int v = 0; v < 4; v++) {  // lane: token 16 i + 4 g + v, expert 16 jj + r
                const int o = (wave * TM + 16 * i + 4 * g + v) * TN + 16 * jj + r;
                fC[o] = acc[i][jj][v];
                fS[o] = sab[i][jj][v];
            }
    if (g == 0) {
#pragma unroll
        for (int i = 0; i < TM16; i++) fQ[wave * TM + 16 * i + r] = s2[i];
    }
    if (lane < TN) fW[wave * TN + lane] = a.Wn[(int64_t)min(e0 + lane, a.E - 1) * RM_NW + wave];
    __syncthreads();
    // each row's scale as CpuRef.RmsNorm forms it (src/CpuRef.cs:183-191): the waves' double sums in a
    // fixed order, certified against the sequential sum (any order of the d non-negative terms lies within
    // (d + 64) 2^-52 of it), else re-summed in index order by this thread (rare; counted)
    static_assert(TM <= 64, "one lane of wave 0 per row");
    if (wave == 0) {
        const int t = min(t0 + lane, a.T - 1);
        float mean = 0.0f, mhi = 0.0f;
        if (lane < TM) {
            double S = 0.0;
            for (int w = 0; w < RM_NW; w++) S += fQ[w * TM + lane];
            mean_ends(S, ((double)a.d + 64.0) * 0x1p-52 * S, 1.0 / (double)a.d, &mean, &mhi);
        }
        // rows the bound leaves open: the sequential sum by the whole wave, one row after another
        for (unsigned long long open = __ballot(lane < TM && mean != mhi); open; open &= open - 1) {
            const int rr = __builtin_ctzll(open), tr = min(t0 + rr, a.T - 1);
            const double q = seq_sum_sq_wave(a.x + (int64_t)tr * a.d, a.d);
            if (lane == rr) mean = (float)(q / (double)a.d);
            if (lane == 0 && blockIdx.y == 0 && t0 + rr < a.T && a.flags) atomicAdd(&a.flags[0], 1);
        }
        if (lane < TM) {
            const float rinv = rms_scale_from_mean(mean, a.eps);
            fR[lane] = rinv;
            if (blockIdx.y == 0 && t0 + lane < a.T) a.xscale[t] = rinv;
        }
    }
    __syncthreads();
    const double sc = (double)(1.0f / (float)__dsqrt_rn((double)a.d));
    const int nbase = a.d / 16 / RM_NW, nextra = a.d / 16 % RM_NW;  // router_range's split
    for (int o = tid; o < TM * TN; o += RM_NW * 64) {
        const int tl = o / TN, el = o % TN, t = t0 + tl, e = e0 + el;
        if (t >= a.T || e >= a.E) continue;
        const double f = (double)fR[tl] * sc;  // rinv / sqrt(d): exact in double
        double O = 0.0, mainb = 0.0, absC = 0.0;
        float cs = 0.0f;
        for (int w = 0; w < RM_NW; w++) {
            const double nw = 16.0 * (nbase + (w < nextra));
            const double C = fC[(w * TM + tl) * TN + el], Sj = fS[(w * TM + tl) * TN + el];
            mainb += nw * fabs(O) + 36.0 * Sj;
            O += C;
            absC += fabs(C);
            cs += sqrtf((float)fQ[w * TM + tl]) * sqrtf(fW[w * TN + el]);  // (its float roundings: inside the 1.03)
        }
        double B = 0x1.08p-24 * f * (mainb + 44.0 * cs) + 0x1p-50 * f * absC + 0x1p-90 * a.d * (1.0 + f);
        if (!(B < 0x1p100)) B = INFINITY;  // also NaN
        const double L = f * O;
        const int64_t te = (int64_t)t * a.E + e;
        a.Lb[te] = L;
        a.Bb[te] = B;
        a.kb[te] = sel_key(L, B, e);
    }
}

template <int TM16, int TN16>
__global__ __launch_bounds__(RM_NW * 64, 1) void k_router_mm(RmArgs a)
{
    extern __shared__ __align__(16) unsigned char rmsm[];  // RmLds<TM16, TN16>::BYTES
    router_mm_tile<TM16, TN16>(a, rmsm);
}

// PRESEL: the selection's inputs are loaded at entry and held in registers through the shared units
// (left out where the register budget is tight)
template <int TYPE, bool PRESEL>
__device__ void gu_wg(const DecArgs& a, unsigned char* smem)
{
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, NT = blockDim.x, NWV = NT >> 6;
    const int nb = a.gu.nb;
    // LDS: [terms | exact-selection arrays and router input] [act rows] [ids, perm, lists, tiles] [scratch]
    const size_t terms_bytes = (size_t)DROWS * nb * 64 * 4, sel_bytes = sel_lds(a.T, a.E, a.d, NT).total;
    unsigned char* un = smem;
    ActL* act = (ActL*)(un + ((std::max(terms_bytes, sel_bytes) + 15) & ~(size_t)15));
    int* s_ids = (int*)(act + DROWS);   // 256
    int* s_perm = s_ids + 256;          // 256
    int* s_cnt = s_perm + 256;          // 260
    int* s_off = s_cnt + 260;           // 260
    int* s_tb = s_off + 260;            // 260
    DecTile* s_tiles = (DecTile*)(s_tb + 260);  // 272
    int* s_misc = (int*)(s_tiles + 272);        // [0] ntiles, [1] any uncertified, [2..17] bad per token
    int* wtot = s_misc + 20;                    // 32
    double* red = (double*)(wtot + 32);         // 17
    unsigned* s_kb = (unsigned*)(red + 17);     // [waves][2][16] selection bounds
    const bool routing = blockIdx.x == gridDim.x - 1;  // the routing workgroup: outputs, no units
    // units: the shared FFN's (token pair, row group) units first, then the expert (tile, row group)
    // units; unit workgroup b takes units b, b + G, b + 2G, ... (G = gridDim.x - 1)
    const int G = gridDim.x - 1;
    const int nsh = a.sgu.rg ? (a.T + DROWS - 1) / DROWS * a.sgu.rg : 0;
    const int total = nsh + a.max_tiles * a.gu.rg;
    int u = routing ? total : (int)blockIdx.x;
    TL_STAMP(a.seq, 1, 0);
    TL_HWID(a.seq, 1, 11);
    // this wave's token's selection inputs (tokens past the waves load theirs at the selection)
    SelIn sin;
    if (PRESEL && wave < a.T) sel_issue(a, wave, sin);
    if (u < nsh) {
        for (; u < nsh; u += G) shared_gu_wg<TYPE>(a, u / a.sgu.rg, u % a.sgu.rg, smem);
        TL_STAMP(a.seq, 1, 1);
        if (u >= total) return;  // uniform: no barriers follow
        __syncthreads();         // the shared units' LDS becomes the selection's
    }
    // one token: every tile's input row is row 0, so its loads go out now, beside the selection's (the
    // router launch wrote it: a cold read that would otherwise start only once the tile is known)
    const bool pre = a.T == 1 && !routing;
    ActIn ain;
    if (pre) act_issue(ain, a.agu, 0, 0, 1, nb);
    if (tid == 0) s_misc[1] = 0;
    __syncthreads();
    TL_STAMP_LANDED(a.seq, 1, 10);
    for (int t = wave; t < a.T; t += NWV) {
        if (!PRESEL || t != wave) sel_issue(a, t, sin);
        const bool cert = wave_topk(a, t, sin, s_ids, s_kb + wave * 32, s_kb + wave * 32 + 16);
        if (lane == 0) {
            s_misc[2 + t] = !cert;
            if (!cert) s_misc[1] = 1;
        }
    }
    TL_STAMP(a.seq, 1, 8);
    __syncthreads();
    TL_STAMP(a.seq, 1, 9);
    const bool exact = s_misc[1] != 0;
    double* sL = (double*)un;
    if (exact) select_exact(a, un, s_ids, s_misc + 2, red, routing);
    int ntiles;
    if (a.T == 1) {
        // one token: tile j is assignment j (the k experts are distinct)
        if (tid < a.k) s_tiles[tid] = DecTile{s_ids[tid], 1, {tid, 0}};
        if (routing) {
            // expert lists: rank of assignment tid in ascending expert order; offsets by counting
            if (tid < a.k) {
                const int e = s_ids[tid];
                int r = 0;
                for (int j = 0; j < a.k; j++) r += s_ids[j] < e;
                s_perm[r] = tid;
            }
            for (int x = tid; x <= a.E; x += NT) {
                int c = 0;
                for (int j = 0; j < a.k; j++) c += s_ids[j] < x;
                s_off[x] = c;
            }
        }
        ntiles = a.k;
        __syncthreads();
    } else {
        build_tiles(a, s_ids, s_cnt, s_off, s_tb, s_perm, s_tiles, s_misc, wtot);
        ntiles = s_misc[0];
    }
    TL_STAMP(a.seq, 1, 2);
    if (routing) {
        const double* Lg = a.Lb;
        const int* bad = s_misc + 2;
        const int E = a.E;
        write_routing(
            a, [&](int t, int e) { return (exact && bad[t]) ? sL[t * E + e] : Lg[(int64_t)t * E + e]; }, s_ids, s_off,
            s_perm, s_tiles, ntiles);
        return;
    }
    for (; u < total; u += G) {
        const int x = u - nsh, tile = x / a.gu.rg, rgi = x % a.gu.rg;
        if (tile >= ntiles) return;  // uniform; the later units of this workgroup lie past the tiles too
        const DecTile tl = s_tiles[tile];
        const int e = tl.e, cnt = min(tl.cnt, DROWS);
        const int tok0 = tl.row[0] / a.k, tok1 = tl.row[cnt > 1 ? 1 : 0] / a.k;
        if (!pre) act_issue(ain, a.agu, tok0, tok1, cnt, nb);  // one token: ain holds row 0 throughout
        __builtin_amdgcn_sched_barrier(0);  // keep the activation loads ahead of the weight loads
        WRegs<TYPE> W;
        load_w<TYPE>(a.gu, clamp_id(e, a.E), rgi, wave, lane, W);  // unconditional (see load_w)
        TL_STAMP(a.seq, 1, 6);
        __syncthreads();  // the exact-selection arrays (first unit) or the last unit's rows are done with
        act_store(ain, cnt, nb, act);
        TL_STAMP(a.seq, 1, 7);
        __syncthreads();
        TL_STAMP(a.seq, 1, 3);
        const float S = rowgroup_chain<TYPE>(W, wave, nb, act, cnt, (float*)un);
        TL_STAMP(a.seq, 1, 4);
        if (wave < cnt) gu_epilogue(S, rgi, a.nf, wave == 0 ? tl.row[0] : tl.row[1], a.g, a.u, a.adn, a.gelu_tab);
    }
    TL_STAMP(a.seq, 1, 5);
}

// NTMAX: the workgroup-size bound the compiler allocates registers for (768 gives the unit loop the
// registers it needs without scratch, and room for the early selection loads; 1024 for the widest rows)
template <int TYPE, int NTMAX>
__global__ __launch_bounds__(NTMAX) void k_dec_gu(DecArgs a)
{
    extern __shared__ __align__(16) unsigned char dsm[];
    gu_wg<TYPE, (NTMAX <= 768)>(a, dsm);  // shared and expert units, or (the last workgroup) the routing outputs
}

// ------------------------------------------------------------------------------ k_dec_down
// Expert workgroups: a tile (from k_dec_gu's workgroup 0) and rpw consecutive row groups, wpr =
// ceil(nb / 8) waves each: yd[a][row] = down_e(gelu(g) * u)[row] for the tile's assignments.  Shared
// workgroups (after the expert ones): the shared FFN's down product.
template <int TYPE>
__global__ __launch_bounds__(1024) void k_dec_down(DecArgs a)
{
    extern __shared__ __align__(16) unsigned char dsm[];
    const int nb = a.dn.nb, wpr = (nb + DBPW - 1) / DBPW, nrgb = (a.dn.rg + a.rpw - 1) / a.rpw;
    const int ne = a.max_tiles * nrgb;
    TL_STAMP(a.seq, 2, 0);
    if ((int)blockIdx.x >= ne) {
        const int s = blockIdx.x - ne;
        shared_dn_wg<TYPE>(a, s / a.sdn.rg, s % a.sdn.rg, dsm);
        TL_STAMP(a.seq, 2, 3);
        return;
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int tile = blockIdx.x / nrgb, g = wave / wpr, wl = wave % wpr;
    const int rgi = (blockIdx.x % nrgb) * a.rpw + g;
    const bool live = g < a.rpw && rgi < a.dn.rg;  // spare waves compute a clamped row group, store nothing
    // one token: tile j is assignment j, so its input row is known before the (cold) tile load
    ActIn ain;
    if (a.T == 1) act_issue(ain, a.adn, min(tile, a.k - 1), min(tile, a.k - 1), 1, nb);
    const int4 tl = *(const int4*)(a.tiles + tile);  // {e, cnt, row0, row1}
    if (tl.x < 0) return;                            // slot past the last tile (uniform)
    const int e = tl.x, cnt = min(tl.y, DROWS);
    ActL* act = (ActL*)dsm;
    float* terms = (float*)(act + DROWS) + (size_t)min(g, a.rpw - 1) * DROWS * nb * 64;
    if (a.T != 1) act_issue(ain, a.adn, tl.z, cnt > 1 ? tl.w : tl.z, cnt, nb);
    __builtin_amdgcn_sched_barrier(0);  // keep the activation loads ahead of the weight loads
    WRegs<TYPE> W;
    load_w<TYPE>(a.dn, clamp_id(e, a.E), min(rgi, a.dn.rg - 1), wl, lane, W);  // unconditional (see load_w)
    act_store(ain, cnt, nb, act);
    __syncthreads();
    TL_STAMP(a.seq, 2, 1);
    const float S = rowgroup_chain<TYPE>(W, live ? wl : wpr, nb, act, cnt, terms);
    TL_STAMP(a.seq, 2, 2);
    const int row = rgi * 64 + lane;
    if (live && wl < cnt && row < a.d) a.yd[(int64_t)(wl == 0 ? tl.z : tl.w) * a.d + row] = S;
    TL_STAMP(a.seq, 2, 3);
}

// ------------------------------------------------------------------------------ k_dec_combine
// Per token (1024 threads): acc = sum_j w_j * yd_j in rank order (src/GemmaCpu.cs:417-418, each term
// rounded then added), out = rmsnorm(shared) * post1 + rmsnorm(acc) * post2 (src/GemmaCpu.cs:384,
// 420-421), and with a residual x += rmsnorm(out) * post_ffw_norm (src/GemmaCpu.cs:355-356).  Every
// load of the token, the residual row included, is issued in one round before the first use (d <= 4096:
// one float4 of four consecutive columns per thread; ranks in groups of 8), and the two branch norms
// share one reduction.
constexpr int CB_NT = 1024, CB_E = 4;

__global__ __launch_bounds__(CB_NT) void k_dec_combine(DecArgs a)
{
    extern __shared__ __align__(16) float cb[];  // acc [d], out [d]
    __shared__ double red[2 * (CB_NT / 64 + 1)];
    const int t = blockIdx.x, tid = threadIdx.x, d = a.d, k = a.k, n4 = d / 4;
    float4* sacc = (float4*)cb;
    float4* so = (float4*)(cb + d);
    const float4* sh = a.shout ? (const float4*)(a.shout + (int64_t)t * d) : nullptr;
    float4* xr = a.xres ? (float4*)(a.xres + (int64_t)t * d) : nullptr;
    const float4* xi = a.xin ? (const float4*)(a.xin + (int64_t)t * d) : xr;  // the residual's source row
    const float4* yd = (const float4*)a.yd + (int64_t)t * k * n4;
    const float4 z4 = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const int ix = min(tid, n4 - 1);  // thread tid: columns 4 tid .. 4 tid + 3 (d <= 4 CB_NT)
    const bool own = tid < n4;
    float4 acc = z4, shv = z4, p1, p2, xv = z4, pf = z4;
    // ranks in groups of 8, every load of a group issued before its first use
    for (int j0 = 0; j0 < k; j0 += 8) {
        float4 yv[8];
        float wj[8];
#pragma unroll
        for (int jj = 0; jj < 8; jj++) wj[jj] = a.w[(int64_t)t * k + min(j0 + jj, k - 1)];
#pragma unroll
        for (int jj = 0; jj < 8; jj++) yv[jj] = yd[(int64_t)min(j0 + jj, k - 1) * n4 + ix];
        if (j0 == 0) {
            if (sh) shv = sh[ix];
            p1 = ((const float4*)a.post1)[ix];
            p2 = ((const float4*)a.post2)[ix];
            if (xr) {
                xv = xi[ix];
                pf = ((const float4*)a.post_ffw)[ix];
            }
        }
#pragma unroll
        for (int jj = 0; jj < 8; jj++)
            if (j0 + jj < k) {
                acc.x += yv[jj].x * wj[jj];
                acc.y += yv[jj].y * wj[jj];
                acc.z += yv[jj].z * wj[jj];
                acc.w += yv[jj].w * wj[jj];
            }
    }
    double s2 = 0.0, s1 = 0.0;
    if (own) {
        sacc[tid] = acc;
        s2 = ((double)acc.x * (double)acc.x + (double)acc.y * (double)acc.y) +
             ((double)acc.z * (double)acc.z + (double)acc.w * (double)acc.w);
        s1 = ((double)shv.x * (double)shv.x + (double)shv.y * (double)shv.y) +
             ((double)shv.z * (double)shv.z + (double)shv.w * (double)shv.w);
    }
    __syncthreads();
    float m2, m1;
    wg_mean_sq2(s2, s1, cb, sh ? (const float*)sh : nullptr, d, red, a.flags, &m2, &m1);
    const float sc2 = rms_scale_from_mean(m2, a.eps);
    const float sc1 = sh ? rms_scale_from_mean(m1, a.eps) : 0.0f;
    acc = sacc[ix];  // from LDS: not held in registers across the means' fallback
    float4 ov;
    ov.x = (sh ? shv.x * sc1 * p1.x : 0.0f) + acc.x * sc2 * p2.x;
    ov.y = (sh ? shv.y * sc1 * p1.y : 0.0f) + acc.y * sc2 * p2.y;
    ov.z = (sh ? shv.z * sc1 * p1.z : 0.0f) + acc.z * sc2 * p2.z;
    ov.w = (sh ? shv.w * sc1 * p1.w : 0.0f) + acc.w * sc2 * p2.w;
    double s3 = 0.0;
    if (own) {
        ((float4*)(a.out + (int64_t)t * d))[tid] = ov;
        so[tid] = ov;
        s3 = ((double)ov.x * (double)ov.x + (double)ov.y * (double)ov.y) +
             ((double)ov.z * (double)ov.z + (double)ov.w * (double)ov.w);
    }
    if (xr) {
        __syncthreads();
        const float sc3 = rms_scale_from_mean(wg_mean_sq(s3, cb + d, d, red, a.flags), a.eps);
        if (own)
            xr[tid] = make_float4(xv.x + ov.x * sc3 * pf.x, xv.y + ov.y * sc3 * pf.y, xv.z + ov.z * sc3 * pf.z,
                                  xv.w + ov.w * sc3 * pf.w);
    }
}

// ------------------------------------------------------------------------------ launchers

static MatD mat_d(const QMat* q)
{
    MatD m{};
    if (!q || !q->payload) return m;
    m.pay = q->payload;
    m.mat_pay = q->mat_pay_stride();
    m.rg_pay = q->rg_pay;
    m.sc_off = q->sc8_off();
    m.rg = q->rg;
    m.nb = q->nb;
    m.nb8 = (q->nb + 7) / 8;
    m.rows = q->rows;
    return m;
}

static int waves_for(int nb) { return (nb + DBPW - 1) / DBPW; }

// block sizes: a row-group workgroup has one wave per 8 blocks (at least 4 where the selection and the
// lists run); the router has d / 4 threads; a down workgroup holds rpw expert row groups, as many as
// fit the shared down's workgroup size
static int nt_gu(const DecLayerH& h)
{
    int nw = std::max(4, waves_for(h.gu->nb));
    if (h.sgu) nw = std::max(nw, waves_for(h.sgu->nb));
    return 64 * nw;
}

static int nw_down(const DecLayerH& h) { return std::max(waves_for(h.dn->nb), h.sdn ? waves_for(h.sdn->nb) : 0); }
static int rpw_down(const DecLayerH& h) { return nw_down(h) / waves_for(h.dn->nb); }

static DecArgs dec_args(const DecLayerH& h)
{
    DecArgs a{};
    a.T = h.T;
    a.d = h.d;
    a.E = h.E;
    a.k = h.k;
    a.nf = h.nf;
    a.nff = h.sgu ? h.nff : 0;
    a.rule = h.rule;
    a.max_tiles = h.max_tiles;
    a.seq = h.seq;
    a.eps = h.eps;
    a.x = h.x;
    a.xscale = h.xscale;
    a.W = h.W;
    a.gis = h.gis;
    a.ds = h.ds;
    a.pre2 = h.pre2;
    a.post1 = h.post1;
    a.post2 = h.post2;
    a.fnorm = h.fnorm;
    a.post_ffw = h.post_ffw;
    a.gu = mat_d(h.gu);
    a.dn = mat_d(h.dn);
    a.sgu = mat_d(h.sgu);
    a.sdn = mat_d(h.sdn);
    a.agu = h.agu;
    a.ash = h.sgu ? h.ash : Act{};
    a.rpw = rpw_down(h);
    a.Lb = h.Lb;
    a.Bb = h.Bb;
    a.kb = (uint4*)h.kb;
    a.cbad = h.bad;
    a.ids = h.ids;
    a.w = h.w;
    a.logits = h.logits;
    a.offsets = h.offsets;
    a.perm = h.perm;
    a.tiles = h.tiles;
    a.g = h.g;
    a.u = h.u;
    a.adn = h.adn;
    a.yd = h.yd;
    a.shg = h.shg;
    a.shu = h.shu;
    a.asd = h.asd;
    a.shout = h.sgu ? h.shout : const_cast<float*>(h.shared_in);
    a.out = h.out;
    a.xres = h.xres;
    a.xin = h.xin;
    a.gelu_tab = h.gelu_tab;
    a.flags = h.flags;
    return a;
}

static size_t gu_lds(const DecLayerH& h)
{
    const size_t un = (std::max((size_t)DROWS * h.gu->nb * 64 * 4, sel_lds(h.T, h.E, h.d, nt_gu(h)).total) + 15) & ~(size_t)15;
    const size_t ex = un + sizeof(ActL) * DROWS + (256 * 2 + 260 * 3) * 4 + 272 * sizeof(DecTile) + (20 + 32) * 4 + 17 * 8 +
                      16 * 32 * 4;
    const size_t sh = h.sgu ? sizeof(ActL) * DROWS + (size_t)DROWS * h.sgu->nb * 64 * 4 : 0;
    return std::max(ex, sh);
}

static size_t down_lds(const DecLayerH& h)
{
    const size_t ex = sizeof(ActL) * DROWS + (size_t)rpw_down(h) * DROWS * h.dn->nb * 64 * 4;
    const size_t sh = h.sdn ? sizeof(ActL) * DROWS + (size_t)DROWS * h.sdn->nb * 64 * 4 : 0;
    return std::max(ex, sh);
}

template <class K>
static void raise_lds(K kernel, size_t bytes)
{
    (void)hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

bool dec_supported(const DecLayerH& h)
{
    if (h.d > 4096 || h.d % 256 || h.gu->nb > DMAXNB || h.gu->nb > 32 * h.E || h.dn->nb > DMAXNB || h.E > 256 || h.T * h.k > 256) return false;
    if (h.sgu && (h.sgu->nb > DMAXNB || h.sdn->nb > DMAXNB)) return false;
    if (nt_gu(h) < std::max(h.E, h.T * h.k)) return false;  // build_tiles: a thread per expert and assignment
    return gu_lds(h) <= 160 * 1024 && down_lds(h) <= 160 * 1024;
}

template <template <int> class KT>
static void launch_typed(const DecLayerH& h, dim3 grid, dim3 block, size_t lds, hipStream_t st, const DecArgs& a)
{
    if (h.gu->type == PHX_Q4_0_DEV) {
        raise_lds(KT<PHX_Q4_0_DEV>::fn, lds);
        launch(KT<PHX_Q4_0_DEV>::fn, grid, block, (uint32_t)lds, st, a);
    } else {
        raise_lds(KT<PHX_Q8_0_DEV>::fn, lds);
        launch(KT<PHX_Q8_0_DEV>::fn, grid, block, (uint32_t)lds, st, a);
    }
}
template <int T> struct KGu { static constexpr auto fn = k_dec_gu<T, 768>; };
template <int T> struct KGuW { static constexpr auto fn = k_dec_gu<T, 1024>; };
template <int T> struct KDown { static constexpr auto fn = k_dec_down<T>; };

static auto route_mx_kernel(int per)
{
    switch (per) {
    case 1: return KRouteMx<1>::fn;
    case 2: return KRouteMx<2>::fn;
    case 3: return KRouteMx<3>::fn;
    case 4: return KRouteMx<4>::fn;
    case 5: return KRouteMx<5>::fn;
    case 6: return KRouteMx<6>::fn;
    case 7: return KRouteMx<7>::fn;
    case 8: return KRouteMx<8>::fn;
    case 9: return KRouteMx<9>::fn;
    case 10: return KRouteMx<10>::fn;
    case 11: return KRouteMx<11>::fn;
    case 12: return KRouteMx<12>::fn;
    case 13: return KRouteMx<13>::fn;
    case 14: return KRouteMx<14>::fn;
    case 15: return KRouteMx<15>::fn;
    default: return KRouteMx<16>::fn;
    }
}

void launch_dec_route(hipStream_t st, const DecLayerH& h)
{
    const int per = route_per(h.T, h.E, h.d), nt = h.d / per;
    // a workgroup per token and RT_RX experts, where its 8-lane groups cover the token's input blocks
    if ((int64_t)h.T * h.E > 1024 && h.E % RT_RX == 0 && h.d / 32 <= nt / 8 * (h.E / RT_RX)) {
        const size_t lds = (size_t)(2 + RT_RX) * route_row_floats(h.d, nt) * 4;
        const auto kr = route_mx_kernel(per);
        raise_lds(kr, lds);
        launch(kr, dim3(h.T * (h.E / RT_RX)), dim3(nt), (uint32_t)lds, st, dec_args(h));
        return;
    }
    const size_t lds = (size_t)3 * route_row_floats(h.d, nt) * 4;
    const auto kr = route_kernel(per);
    raise_lds(kr, lds);
    launch(kr, dim3(h.T * h.E), dim3(nt), (uint32_t)lds, st, dec_args(h));
}

void launch_cert_select(hipStream_t st, const DecLayerH& h)
{
    const DecArgs a = dec_args(h);
    if (cert_select_one_launch(h)) {  // a workgroup per token in at most two rounds: one launch
        const size_t lds1 = sel_lds(1, h.E, h.d, CF_NT, CF_P).total;
        raise_lds(k_cert_select_one, lds1);
        launch(k_cert_select_one, dim3(h.T), dim3(CF_NT), (uint32_t)lds1, st, a);
        return;
    }
    launch(k_cert_select, dim3((h.T + CS_TPW - 1) / CS_TPW), dim3(64 * CS_TPW), 0, st, a);
    // the marked tokens: at most one per compute unit at a time
    const size_t lds = sel_lds(1, h.E, h.d, CF_NT, CF_P).total;
    raise_lds(k_cert_fallback, lds);
    launch(k_cert_fallback, dim3(std::min(h.T, std::max(h.ncu, 1))), dim3(CF_NT), (uint32_t)lds, st, a);
}

template <int A, int B> struct KRm { static constexpr auto fn = k_router_mm<A, B>; };

bool router_mm_supported(int T, int d, int E)
{
    return d % 16 == 0 && d / 16 >= RM_NW && E <= 256 && (int64_t)T * d * 4 < ((int64_t)1 << 31) &&
           (int64_t)E * d * 4 < ((int64_t)1 << 31);
}

void launch_router_mm(hipStream_t st, int T, int d, int E, float eps, const float* x, const float* Ws, const float* Wn,
                      float* xscale, double* Lb, double* Bb, uint32_t* kb, int* cbad, int* flags)
{
    const RmArgs a{T, d, E, eps, x, Ws, Wn, xscale, Lb, Bb, (uint4*)kb, cbad, flags};
    // 32 x 32 tiles where they still give a workgroup per compute unit, 16 x 16 below
    if ((int64_t)((T + 31) / 32) * ((E + 31) / 32) >= 256) {
        using RG = RmLds<2, 2>;
        raise_lds(KRm<2, 2>::fn, RG::BYTES);
        launch(KRm<2, 2>::fn, dim3((T + 31) / 32, (E + 31) / 32), dim3(RM_NW * 64), (uint32_t)RG::BYTES, st, a);
    } else {
        using RG = RmLds<1, 1>;
        raise_lds(KRm<1, 1>::fn, RG::BYTES);
        launch(KRm<1, 1>::fn, dim3((T + 15) / 16, (E + 15) / 16), dim3(RM_NW * 64), (uint32_t)RG::BYTES, st, a);
    }
}

void launch_dec_route_fused(hipStream_t st, const DecLayerH& prev, const DecLayerH& h)
{
    const size_t lds = ((size_t)3 * route_row_floats(h.d, route_threads(h.d)) + 2 * (h.d + 4)) * 4;
    const auto kf = k_dec_route_fused;
    raise_lds(kf, lds);
    CombArgs cb;
    cb.d = prev.d;
    cb.k = prev.k;
    cb.seq = h.seq;
    cb.eps = prev.eps;
    cb.w = prev.w;
    cb.yd = prev.yd;
    cb.shout = prev.sgu ? prev.shout : prev.shared_in;
    cb.post1 = prev.post1;
    cb.post2 = prev.post2;
    cb.post_ffw = prev.post_ffw;
    cb.xin = prev.xin;
    cb.out = prev.out;
    cb.xres = prev.xres;
    cb.flags = prev.flags;
    launch(kf, dim3(h.T * h.E), dim3(route_threads(h.d)), (uint32_t)lds, st, cb, dec_args(h));
}

void launch_dec_gu(hipStream_t st, const DecLayerH& h)
{
    const int nsh = h.sgu ? (h.T + DROWS - 1) / DROWS * h.sgu->rg : 0;
    const int units = nsh + h.max_tiles * h.gu->rg;
    const dim3 grid(std::min(units, std::max(1, h.ncu)) + 1);
    if (nt_gu(h) <= 768) launch_typed<KGu>(h, grid, dim3(nt_gu(h)), gu_lds(h), st, dec_args(h));
    else launch_typed<KGuW>(h, grid, dim3(nt_gu(h)), gu_lds(h), st, dec_args(h));
}

void launch_dec_down(hipStream_t st, const DecLayerH& h)
{
    const int rpw = rpw_down(h), nrgb = (h.dn->rg + rpw - 1) / rpw;
    const int nsh = h.sdn ? (h.T + DROWS - 1) / DROWS * h.sdn->rg : 0;
    launch_typed<KDown>(h, dim3(h.max_tiles * nrgb + nsh), dim3(64 * nw_down(h)), down_lds(h), st, dec_args(h));
}

// The general path's combine (any T): the same kernel over the general path's rows; per token acc =
// sum_j yd[t*k+j] * w_j in rank order (src/GemmaCpu.cs:418, each term rounded then added),
// out = rmsnorm(shared) * post1 + rmsnorm(acc) * post2 (src/GemmaCpu.cs:384,420-421), and with xres
// x += rmsnorm(out) * post_ffw_norm in place (src/GemmaCpu.cs:355-356).
void launch_combine(hipStream_t st, int T, int d, int k, float eps, const float* yd, const float* w, const float* shared,
                    const float* post1, const float* post2, float* out, float* xres, const float* post_ffw, int* flags)
{
    if (d > CB_E * CB_NT) {
        launch_combine_wide(st, T, d, k, eps, yd, w, shared, post1, post2, out, xres, post_ffw, flags);
        return;
    }
    DecArgs a{};
    a.T = T;
    a.d = d;
    a.k = k;
    a.eps = eps;
    a.yd = const_cast<float*>(yd);
    a.w = const_cast<float*>(w);
    a.shout = const_cast<float*>(shared);
    a.post1 = post1;
    a.post2 = post2;
    a.out = out;
    a.xres = xres;
    a.post_ffw = post_ffw;
    a.flags = flags;
    launch(k_dec_combine, dim3(T), dim3(CB_NT), (uint32_t)((size_t)2 * d * 4), st, a);
}

void launch_dec_combine(hipStream_t st, const DecLayerH& h)
{
    launch(k_dec_combine, dim3(h.T), dim3(CB_NT), (uint32_t)((size_t)2 * h.d * 4), st, dec_args(h));
}

}  // namespace phx

#ifdef PHX_TIMELINE
// the instrumented build's clock-stamp table [seq][kind][slot][workgroup], 100 MHz ticks (0: no stamp)
extern "C" __attribute__((visibility("default"))) int phxdbg_timeline(unsigned long long* host, size_t n, int clear)
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
