// Decode-shaped MoE FFN kernels (a few tokens, T <= 16): four launches per layer.
//   k_route_dec    router logits (certified), the quantized expert / shared-FFN inputs, then in the
//                  last workgroup: top-k, weights and the expert lists
//   k_dec_mm<0>    gate|up of the routed experts and of the shared FFN; epilogue: gelu(g) * u and
//                  its Q8_0 quantization (the down input)
//   k_dec_mm<1>    down of the routed experts and of the shared FFN
//   k_combine_dec  rank-ordered combine, branch norms, optional residual
// Arithmetic follows the reference CPU path (src/GemmaCpu.cs:376-422) as in kernels.hip; the router
// logits are the one quantity certified rather than replayed (see k_route_dec).
#include <algorithm>

#include "device_common.h"

namespace phx {

// Q8_0 of 32 values held one per lane of a 32-lane half (CpuRef.QuantizeQ8_0, src/CpuRef.cs:49-62):
// returns q; *dval and *sum (fp16 scale value and block sum) are valid in every lane of the half.
__device__ __forceinline__ int q8_0_half(float x, float* dval, int* sum)
{
    const float amax = half_max_f(fabsf(x));
    const float dd = amax / 127.0f;
    const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
    const int q = (int)roundf(x * id);
    *dval = h2f(f2h_bits(dd));
    *sum = half_sum_i(q);
    return q;
}

// ------------------------------------------------------------------------------ router (decode)
// One wave per (token, expert).  The reference logit is the sequential float sum of the rounded
// products p_i = fl(W[e][i] * m_i) (src/GemmaCpu.cs:390-395).  The wave forms the same p_i, sums
// them in double (L), and bounds the reference's accumulated rounding:
//   |S_ref - L| <= 2^-24 * sum_k |S_k| / (1 - n 2^-24)  (+ slack for the double arithmetic),
// S_k the exact prefix sums (a wave scan).  The last workgroup ranks the experts by L and accepts
// the order if every chosen expert's interval lies strictly above every later expert's; otherwise
// the experts whose intervals reach the chosen ones are recomputed as the reference's float chains
// and ranked exactly.  Ids are therefore always the reference's; weights use (float)L for certified
// tokens (within ~1e-6 of the reference's logit) and the exact logits otherwise.
// The same launch also writes the Q8_0 expert input n = x * scale * pre_ffw_norm_2 (and the shared
// FFN input with ffn_norm): workgroup (bx, t) quantizes every (8 * gridDim.x)-th 32-block of token t.
struct RouteDecArgs {
    int T, d, E, k, rule, A, max_tiles;
    float eps;
    const float* x;
    const float* W;       // [E][d] row-major (ffn_gate_inp.weight)
    const float* gis;     // ffn_gate_inp.scale
    const float* ds;      // ffn_down_exps.scale
    const float* pre2;    // pre_ffw_norm_2
    const float* fnorm;   // ffn_norm (shared FFN input) or null
    Act act_gu, act_sh;
    double* Lb;           // [T][E]
    double* Bb;           // [T][E]
    int* counter;         // zero between launches
    int* ids;
    float* w;
    float* logits;
    int* offsets;
    int* perm;
    DecTile* tiles;
    int* ntiles;
    int* flags;           // [0] norm fallbacks, [1] router fallbacks
};

constexpr int RT_PER = 16;        // elements per lane (d <= 4096, 256 lanes)
typedef __attribute__((address_space(3))) void* lds_void_t;
typedef __attribute__((address_space(1))) void* glb_void_t;

__device__ __forceinline__ double ld_agent(const double* p)
{
    unsigned long long v = __hip_atomic_load((const unsigned long long*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return __longlong_as_double((long long)v);
}

__device__ __forceinline__ void st_agent(double* p, double v)
{
    __hip_atomic_store((unsigned long long*)p, (unsigned long long)__double_as_longlong(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// exact reference logit of expert e for token t (src/GemmaCpu.cs:389-395)
__device__ float exact_logit(const float* x, const float* W, const float* gis, int d, int t, int e, float rinv, float sc)
{
    const float* xr = x + (int64_t)t * d;
    const float* wr = W + (int64_t)e * d;
    float s = 0.0f;
    for (int i = 0; i < d; i += 4) {
        const float4 xv = *(const float4*)(xr + i), gv = *(const float4*)(gis + i), wv = *(const float4*)(wr + i);
        s += wv.x * (xv.x * rinv * sc * gv.x);
        s += wv.y * (xv.y * rinv * sc * gv.y);
        s += wv.z * (xv.z * rinv * sc * gv.z);
        s += wv.w * (xv.w * rinv * sc * gv.w);
    }
    return s;
}

// One workgroup per (expert e, token t): x_t, the router scale and W[e] staged in LDS, then each of
// the 256 lanes takes d / 256 consecutive indices; the double sum, its prefix sums (a wave scan
// plus the four wave totals) and the bound terms follow the layout above.
__global__ __launch_bounds__(256) void k_route_dec(RouteDecArgs a)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, tid = threadIdx.x;
    const int e = blockIdx.x, t = blockIdx.y;
    extern __shared__ __align__(16) unsigned char rsm[];
    __shared__ int s_last, s_bad[16];
    __shared__ double red[8], wsum[4], wA[4], wP[4], s_seq;
    __shared__ int s_ids[256], s_perm[256];
    __shared__ int s_cnt[PHX_MAX_EXPERTS_DEV + 1], s_off[PHX_MAX_EXPERTS_DEV + 1], s_tb[PHX_MAX_EXPERTS_DEV + 1];
    const float sc = 1.0f / (float)__dsqrt_rn((double)a.d);
    const float* xr = a.x + (int64_t)t * a.d;
    const int d = a.d;

    // ---- x_t, the router scale and W[e] into LDS (direct global -> LDS loads, 16 B per lane,
    // every load in flight at once; each wave fills 64 consecutive float4 per instruction)
    float* sx = (float*)rsm;
    float* sg = sx + d;
    float* sw = sg + d;
    // the norm weight of this thread's first quantization slot (see below), loaded beside the staging
    const int nin = a.fnorm ? 2 : 1, q_p0 = e * 8 + (tid >> 5);
    float nw0 = 0.0f;
    if (q_p0 < (d / 32) * nin) {
        const int b = q_p0 / nin;
        nw0 = (q_p0 - b * nin ? a.fnorm : a.pre2)[b * 32 + (tid & 31)];
    }
    {
        const int n4 = d / 4;
        const float4* srcs[3] = {(const float4*)xr, (const float4*)a.gis, (const float4*)(a.W + (int64_t)e * d)};
#pragma unroll
        for (int r = 0; r < 3; r++) {
            float4* dst = (float4*)(sx + r * d);
            for (int q = 0; q * 256 < n4; q++) {
                const int i = q * 256 + tid;
                if (i < n4)
                    __builtin_amdgcn_global_load_lds((glb_void_t)(srcs[r] + i), (lds_void_t)(dst + q * 256 + wave * 64), 16, 0,
                                                     0);
            }
        }
        __builtin_amdgcn_s_waitcnt(0);
    }
    __syncthreads();
    // ---- the lane's contiguous chunk of d / 256 indices (d % 256 == 0)
    const int per = d / 256, c0 = tid * per;
    // certified mean of squares of x_t: every workgroup of the token forms the same sum in the same order
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < RT_PER; j++)
        if (j < per) {
            const double v = (double)sx[c0 + j];
            s += v * v;
        }
    s = wave_sum_dpp(s);
    if (lane == 0) red[wave] = s;
    __syncthreads();
    const double S = (red[0] + red[1]) + (red[2] + red[3]);
    const double Bs = ((double)d + per + 256.0) * 0x1p-53 * S * 2.0;
    float mean = (float)((S - Bs) / (double)d);
    if (mean != (float)((S + Bs) / (double)d)) {  // uniform: S is the same in every thread
        if (tid == 0) {
            double q = 0.0;
            for (int i = 0; i < d; i++) q += (double)sx[i] * (double)sx[i];
            s_seq = q;
            if (a.flags && e == 0) atomicAdd(a.flags, 1);
        }
        __syncthreads();
        mean = (float)(s_seq / (double)d);
    }
    const float rinv = rms_scale_from_mean(mean, a.eps);  // also the RmsNorm scale of x_t
    {
        // p_i = fl(W[e][i] * m_i), m_i = ((x_i * rinv) * sc) * s_i (src/GemmaCpu.cs:389,394)
        float pv[RT_PER];
        double loc = 0.0, P = 0.0;
#pragma unroll
        for (int j = 0; j < RT_PER; j++) {
            if (j < per) {
                pv[j] = sw[c0 + j] * (sx[c0 + j] * rinv * sc * sg[c0 + j]);
                loc += (double)pv[j];
                P += fabs((double)pv[j]);
            } else {
                pv[j] = 0.0f;
            }
        }
        const double inc = wave_incl_scan_dpp(loc);
        if (lane == 63) wsum[wave] = inc;
        __syncthreads();
        double base = 0.0;
        for (int w = 0; w < wave; w++) base += wsum[w];
        double acc = base + (inc - loc);  // exclusive prefix (within the double slack of the bound)
        double A = 0.0;
#pragma unroll
        for (int j = 0; j < RT_PER; j++)
            if (j < per) {
                acc += (double)pv[j];
                A += fabs(acc);
            }
        A = wave_sum_dpp(A);
        P = wave_sum_dpp(P);
        if (lane == 0) {
            wA[wave] = A;
            wP[wave] = P;
        }
        __syncthreads();
        if (tid == 0) {
            const double L = ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3];
            const double As = (wA[0] + wA[1]) + (wA[2] + wA[3]), Ps = (wP[0] + wP[1]) + (wP[2] + wP[3]);
            st_agent(&a.Lb[(int64_t)t * a.E + e], L);
            st_agent(&a.Bb[(int64_t)t * a.E + e], 0x1p-24 * As * 1.001 + 0x1p-45 * Ps);
        }
    }

    // ---- quantized expert input (and shared FFN input) of token t: one 32-lane half per (block, input),
    // spread over the E workgroups of the token
    {
        const int nbK = d / 32, l32 = tid & 31;
        for (int p = q_p0; p < nbK * nin; p += a.E * 8) {
            const int b = p / nin, which = p - b * nin;
            const int i = b * 32 + l32;
            const float nwv = p == q_p0 ? nw0 : (which ? a.fnorm : a.pre2)[i];
            const Act& o = which ? a.act_sh : a.act_gu;
            float dval;
            int sum;
            const int q = q8_0_half(sx[i] * rinv * nwv, &dval, &sum);
            o.q[(int64_t)t * o.qstride + i] = (int8_t)q;
            if (l32 == 0) {
                o.d[(int64_t)t * o.dstride + b] = dval;
                o.s[(int64_t)t * o.sstride + b] = sum;
            }
        }
    }

    // ---- hand-off to the last workgroup: the barrier orders every wave's stores before thread 0's
    // agent-scope release increment; the workgroup that completes the count acquires.
    __syncthreads();
    if (tid == 0) {
        const int total = gridDim.x * gridDim.y;
        const int prev = __hip_atomic_fetch_add(a.counter, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        s_last = prev == total - 1;
    }
    __syncthreads();
    if (!s_last) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");

    const int TE = a.T * a.E;
    double* sL = (double*)rsm;
    double* sB = sL + TE;
    unsigned* s_key = (unsigned*)(sB + TE);
    short* s_rank = (short*)(s_key + TE);
    char* s_amb = (char*)(s_rank + TE);
    for (int i = tid; i < TE; i += 256) {
        sL[i] = ld_agent(&a.Lb[i]);
        sB[i] = ld_agent(&a.Bb[i]);
    }
    if (tid < 16) s_bad[tid] = 0;
    __syncthreads();
    // selection: the rank of every (token, expert) from all pairs in LDS (one to two threads per
    // pair) by a 32-bit key: the order-preserving bits of (float)L with the low 8 bits replaced by
    // 255 - expert, so keys are distinct and ties go to the lower index.  The order is then certified
    // per token if each chosen expert's lower end lies above the upper ends of every expert ranked
    // after it.  An order the key gets wrong (logits within 256 float ulps) is never certified, since
    // certification compares the intervals themselves; such tokens take the exact path below.
    for (int i = tid; i < TE; i += 256) {
        const int ex = i % a.E;
        s_key[i] = (sortable_f32((float)sL[i]) & ~0xFFu) | (unsigned)(255 - ex);
    }
    __syncthreads();
    {
        int split = 1;  // threads per pair: a power of two, split * TE <= 256
        while (split < 64 && split * 2 * TE <= 256) split *= 2;
        const int part = tid % split, chunk = (a.E + split - 1) / split;
        for (int i = tid / split; i < TE; i += 256 / split) {
            const int tt = i / a.E;
            const unsigned my = s_key[i];
            const unsigned* kr = s_key + tt * a.E;
            const int c0 = part * chunk, c1 = min(a.E, c0 + chunk);
            int r = 0, c = c0;
            for (; c + 8 <= c1; c += 8) {  // eight keys in flight per step
                const unsigned k0 = kr[c], k1 = kr[c + 1], k2 = kr[c + 2], k3 = kr[c + 3], k4 = kr[c + 4], k5 = kr[c + 5],
                               k6 = kr[c + 6], k7 = kr[c + 7];
                r += (int)(k0 > my) + (int)(k1 > my) + (int)(k2 > my) + (int)(k3 > my) + (int)(k4 > my) + (int)(k5 > my) +
                     (int)(k6 > my) + (int)(k7 > my);
            }
            for (; c < c1; c++) r += kr[c] > my;
            for (int o = 1; o < split; o <<= 1) r += __shfl_xor(r, o, 64);
            if (part == 0) s_rank[i] = (short)min(r, a.k + 1);
        }
    }
    __syncthreads();
    for (int i = tid; i < TE; i += 256)
        if (s_rank[i] < a.k) s_ids[(i / a.E) * a.k + s_rank[i]] = i % a.E;
    __syncthreads();
    for (int tt = wave; tt < a.T; tt += 4) {
        const double* Lr = sL + tt * a.E;
        const double* Br = sB + tt * a.E;
        const short* Rr = s_rank + tt * a.E;
        double hun = -INFINITY;
        bool fin = true;
        for (int ex = lane; ex < a.E; ex += 64) {
            const double Lq = Lr[ex], Bq = Br[ex];
            if (!(isfinite(Lq) && isfinite(Bq))) fin = false;
            if (Rr[ex] >= a.k) hun = fmax(hun, Lq + Bq);
        }
        hun = wave_max_dpp(hun);
        const bool act = lane < a.k;
        const int ej = act ? s_ids[tt * a.k + lane] : 0;
        const double lo_j = act ? Lr[ej] - Br[ej] : INFINITY, hi_j = act ? Lr[ej] + Br[ej] : -INFINITY;
        // suffix maximum over the later ranks (lanes above), then the unchosen experts
        double suf = hi_j;
        for (int o = 1; o < 16; o <<= 1) {
            const double up = __shfl_down(suf, o, 64);
            if (lane + o < 16) suf = fmax(suf, up);
        }
        const double later = fmax(hun, lane + 1 < 16 ? __shfl_down(suf, 1, 64) : -INFINITY);
        const bool cert = __all(fin && (!act || lo_j > later));
        if (lane == 0) s_bad[tt] = !cert;
    }
    __syncthreads();
    // uncertified tokens: exact chains for every expert that can reach the chosen ones
    for (int tt = 0; tt < a.T; tt++) {
        if (!s_bad[tt]) continue;  // uniform: an LDS value read after a barrier
        if (tid == 0) atomicAdd(&a.flags[1], 1);
        const float rinv_t = rms_scale_from_mean(mean_sq_cert<256>(a.x + (int64_t)tt * a.d, a.d, red, a.flags), a.eps);
        double minlo = INFINITY;
        bool nonfinite = false;
        for (int b = 0; b < a.E; b++) {
            const int j = tt * a.E + b;
            if (!(isfinite(sL[j]) && isfinite(sB[j]))) nonfinite = true;
            if (s_rank[j] < a.k) minlo = fmin(minlo, sL[j] - sB[j]);
        }
        __syncthreads();
        for (int b = tid; b < a.E; b += 256) {
            const int j = tt * a.E + b;
            const bool amb = nonfinite || s_rank[j] < a.k || sL[j] + sB[j] >= minlo;
            s_amb[j] = amb;
            if (amb) sL[j] = (double)exact_logit(a.x, a.W, a.gis, a.d, tt, b, rinv_t, sc);  // the others cannot be chosen
        }
        __syncthreads();
        for (int b = tid; b < a.E; b += 256) {
            const int j = tt * a.E + b;
            const double my = s_amb[j] ? sel_key(sL[j]) : -INFINITY;
            int r = 0;
            for (int c = 0; c < a.E; c++) {
                const int jc = tt * a.E + c;
                r += sel_beats(s_amb[jc] ? sel_key(sL[jc]) : -INFINITY, c, my, b);
            }
            s_rank[j] = (short)r;
        }
        __syncthreads();
    }
    // ids, logits (debug: certified L rounded, or exact), weights (src/GemmaCpu.cs:406-407,417)
    for (int i = tid; i < TE; i += 256) {
        const int tt = i / a.E, ex = i - tt * a.E;
        const int r = s_rank[i];
        if (r < a.k) s_ids[tt * a.k + r] = ex;
        a.logits[i] = (float)sL[i];
    }
    __syncthreads();
    const int n = a.T * a.k;
    const bool fast_lists = n <= 64;  // one wave builds the lists while the others form the weights
    // weights: one lane per (token, rank j); waves take tokens in turn (waves 0-2 beside the list wave)
    {
        const int nw = fast_lists ? 3 : 4;
        for (int tt = wave; wave < nw && tt < a.T; tt += nw) {
            const int j = lane;
            const bool act = j < a.k;
            const int id = act ? s_ids[tt * a.k + j] : 0;
            const float selj = act ? (float)sL[tt * a.E + id] : 0.0f;
            const float sel0 = __shfl(selj, 0, 64);
            // p_0 = exp(0) = 1 exactly, so the CPU's in-place rule uses 1 for every later term
            const float top = (a.rule == 1 && j > 0) ? 1.0f : sel0;
            const float pj = act ? (float)exp((double)(selj - top)) : 0.0f;
            double sum = 0.0;
            for (int q = 0; q < a.k; q++) sum += (double)__shfl(pj, q, 64);  // in rank order
            if (act) {
                a.ids[(int64_t)tt * a.k + j] = id;
                a.w[(int64_t)tt * a.k + j] = (float)((double)pj / sum) * a.ds[id];
            }
        }
    }
    if (fast_lists) {
        if (wave == 3) {
            // lane i = assignment i (token i / k, rank i % k): its place in the stable order by
            // (expert, assignment) is the number of assignments before it in that order
            const bool act = lane < n;
            const int ei = act ? clamp_id(s_ids[lane], a.E) : 0;
            int rank = 0;
            for (int j = 0; j < n; j++) {
                const int ej = clamp_id(s_ids[j], a.E);
                rank += (ej < ei) || (ej == ei && j < lane);
            }
            if (act) {
                a.perm[rank] = lane;
                s_perm[rank] = lane;
            }
            // counts per expert, then exclusive scans of counts and tile counts (4 experts per lane)
            for (int x = lane; x <= a.E; x += 64) s_cnt[x] = 0;
            __builtin_amdgcn_wave_barrier();
            if (act) atomicAdd(&s_cnt[ei], 1);
            __builtin_amdgcn_wave_barrier();
            int c[4], tc[4], sc1 = 0, sc2 = 0;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int ex = lane * 4 + q;
                c[q] = ex < a.E ? s_cnt[ex] : 0;
                tc[q] = (c[q] + a.A - 1) / a.A;
                sc1 += c[q];
                sc2 += tc[q];
            }
            int v1 = sc1, v2 = sc2;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int y1 = __shfl_up(v1, o, 64), y2 = __shfl_up(v2, o, 64);
                if (lane >= o) {
                    v1 += y1;
                    v2 += y2;
                }
            }
            int off = v1 - sc1, tb = v2 - sc2;
            const int used = __shfl(v2, 63, 64);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int ex = lane * 4 + q;
                if (ex < a.E) {
                    a.offsets[ex] = off;
                    for (int r = 0; r * a.A < c[q]; r++) {
                        const int st0 = off + r * a.A, m = min(a.A, c[q] - r * a.A);
                        a.tiles[tb + r] = DecTile{ex, m, {s_perm[st0], m > 1 ? s_perm[st0 + 1] : 0}};
                    }
                }
                off += c[q];
                tb += tc[q];
            }
            if (lane == 0) {
                a.offsets[a.E] = n;
                *a.ntiles = used;
            }
            // slots past the last tile carry e = -1: a grouped workgroup reads one slot and stops
            for (int q = used + lane; q < a.max_tiles; q += 64) a.tiles[q] = DecTile{-1, 0, {0, 0}};
        }
        if (tid == 0) __hip_atomic_store(a.counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }

    // ---- expert lists (ascending assignment order) and tiles of <= A assignments
    for (int x = tid; x <= a.E; x += 256) s_cnt[x] = 0;
    __syncthreads();
    int my_e = 0, my_rank = 0;
    if (tid < n) {
        my_e = clamp_id(s_ids[tid], a.E);
        for (int b = 0; b < tid; b++) my_rank += clamp_id(s_ids[b], a.E) == my_e;
        atomicAdd(&s_cnt[my_e], 1);
    }
    __syncthreads();
    // exclusive scans of the counts and of the tile counts (E <= 256: one expert per thread)
    {
        const int c = tid < a.E ? s_cnt[tid] : 0;
        const int tcount = (c + a.A - 1) / a.A;
        int v1 = c, v2 = tcount;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const int y1 = __shfl_up(v1, o, 64), y2 = __shfl_up(v2, o, 64);
            if (lane >= o) { v1 += y1; v2 += y2; }
        }
        __shared__ int wtot1[4], wtot2[4];
        if (lane == 63) { wtot1[wave] = v1; wtot2[wave] = v2; }
        __syncthreads();
        int b1 = 0, b2 = 0;
        for (int w = 0; w < wave; w++) { b1 += wtot1[w]; b2 += wtot2[w]; }
        if (tid < a.E) { s_off[tid] = b1 + v1 - c; s_tb[tid] = b2 + v2 - tcount; }
        if (tid == 0) {
            s_off[a.E] = wtot1[0] + wtot1[1] + wtot1[2] + wtot1[3];
            *a.ntiles = wtot2[0] + wtot2[1] + wtot2[2] + wtot2[3];
        }
        __syncthreads();
    }
    for (int x = tid; x <= a.E; x += 256) a.offsets[x] = s_off[x];
    if (tid < n) {
        a.perm[s_off[my_e] + my_rank] = tid;
        s_perm[s_off[my_e] + my_rank] = tid;
    }
    __syncthreads();
    if (tid < a.E) {
        const int c = s_cnt[tid], base = s_tb[tid];
        for (int q = 0; q * a.A < c; q++) {
            const int st0 = s_off[tid] + q * a.A, m = min(a.A, c - q * a.A);
            a.tiles[base + q] = DecTile{tid, m, {s_perm[st0], m > 1 ? s_perm[st0 + 1] : 0}};
        }
    }
    {
        // slots past the last tile carry e = -1: a grouped workgroup reads one slot and stops
        const int used = s_tb[a.E - 1] + (s_cnt[a.E - 1] + a.A - 1) / a.A;
        for (int q = used + tid; q < a.max_tiles; q += 256) a.tiles[q] = DecTile{-1, 0, {0, 0}};
    }
    if (tid == 0) __hip_atomic_store(a.counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

void launch_route_dec(hipStream_t st, const RouteDecArgsH& h)
{
    RouteDecArgs a{h.T, h.d, h.E, h.k, h.rule, h.A, h.max_tiles, h.eps, h.x, h.W, h.gis, h.ds, h.pre2, h.fnorm, h.act_gu,
                   h.act_sh, h.Lb, h.Bb, h.counter, h.ids, h.w, h.logits, h.offsets, h.perm, h.tiles, h.ntiles, h.flags};
    // staging [3][d] floats, or for the last workgroup L, B (8 B each), key (4 B), rank (2 B), flag (1 B) per (token, expert)
    const size_t lds = std::max((size_t)3 * h.d * sizeof(float), (size_t)h.T * h.E * 23);
    static bool attr = false;
    if (!attr) {
        (void)hipFuncSetAttribute((const void*)k_route_dec, hipFuncAttributeMaxDynamicSharedMemorySize, 3 * 4096 * 4);
        attr = true;
    }
    launch(k_route_dec, dim3(h.E, h.T), dim3(256), lds, st, a);
}

// ------------------------------------------------------------------------------ grouped products (decode)
// Work items: (tile of <= DEC_A assignments of one expert, row group of 64 rows) for the experts,
// then (tile of <= DEC_A tokens, row group) for the dense shared FFN.  The 8 waves each take a
// contiguous slice of the row's blocks with all their weight loads issued at once (lane = row),
// read the activation blocks (wave-uniform) from the Q8_0 buffers, and store the per-block terms
// (float)isum * (d_w * d_x) in LDS; one wave per assignment adds them in block order: the
// reference's float chain (src/CpuRefGemma.cs:27-36, src/CpuRef.cs:106-115).
// Gate|up matrices are repacked in paired row groups (lanes 0-31 gate rows 32g.., lanes 32-63 the
// matching up rows), so the epilogue forms e = gelu(g) * u (src/GemmaCpu.cs:415) for 32 consecutive
// outputs and writes their Q8_0 block, the down input (src/CpuRef.cs:49-62).

constexpr int DEC_A = kDecA;
static_assert(DEC_A == 2, "DecTile holds two assignment rows");

struct DecMat {
    const uint8_t* pay;
    const uint8_t* sc;
    int64_t mat_pay, mat_sc;
    int rg, nb, rows;
    Act in;               // activations (rows: token for gate|up, assignment for down)
    float* out0;          // gate|up: g rows [r][split]; down: y rows [r][rows]
    float* out1;          // gate|up: u rows
    int split;            // gate|up: n_ff (valid outputs per row of g/u)
    Act out_act;          // gate|up: Q8_0 of gelu(g) * u
};

struct DecArgs {
    DecMat m0, m1;        // experts, shared FFN (m1.rg == 0: none)
    const DecTile* tiles;
    int max_tiles;
    int act_div;          // expert activation row = assignment row / act_div
    int T;
    const float* gelu_tab;
};

// NW waves per workgroup, each holding up to MAXB blocks of its lane's row (nb <= NW * MAXB)
template <int MODE, int TYPE, int NW, int MAXB>
__global__ __launch_bounds__(NW * 64) void k_dec_mm(DecArgs a)
{
    constexpr int DEC_NW = NW, DEC_MAXB = MAXB;
    __shared__ float terms[DEC_A][DEC_MAXB * DEC_NW][64];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    constexpr int PAY = TYPE == PHX_Q4_0_DEV ? 16 : 32;

    int which, rgi, e, cnt;
    int orow[DEC_A], arow[DEC_A];
    const int nexp = a.max_tiles * a.m0.rg;
    if ((int)blockIdx.x < nexp) {
        which = 0;
        const int tile = blockIdx.x / a.m0.rg;
        rgi = blockIdx.x % a.m0.rg;
        const int4 tl = *(const int4*)(a.tiles + tile);  // {e, cnt, row0, row1}
        // wave-uniform values: scalar registers, so the activation rows are read with scalar loads
        e = __builtin_amdgcn_readfirstlane(tl.x);
        if (e < 0) return;  // slot past the last tile
        cnt = min(__builtin_amdgcn_readfirstlane(tl.y), DEC_A);
        orow[0] = __builtin_amdgcn_readfirstlane(tl.z);
        orow[1] = __builtin_amdgcn_readfirstlane(tl.w);
        arow[0] = orow[0] / a.act_div;
        arow[1] = orow[1] / a.act_div;
    } else {
        which = 1;
        const int sid = blockIdx.x - nexp;
        const int tile = sid / a.m1.rg;
        rgi = sid % a.m1.rg;
        e = 0;
        const int t0 = tile * DEC_A;
        cnt = min(DEC_A, a.T - t0);
#pragma unroll
        for (int i = 0; i < DEC_A; i++) orow[i] = arow[i] = t0 + i;
    }
    const DecMat M = which ? a.m1 : a.m0;
    const int nb = M.nb;

    // ---- weights: this wave's blocks of the lane's row, all loads issued at once
    const int bpw = (nb + DEC_NW - 1) / DEC_NW;
    const int b0 = wave * bpw, b1 = min(nb, b0 + bpw);
    const uint8_t* wp = M.pay + e * M.mat_pay + ((int64_t)rgi * nb * 64 + lane) * PAY;
    const uint16_t* ws = (const uint16_t*)(M.sc + e * M.mat_sc) + (int64_t)rgi * nb * 64 + lane;
    uint4 wv[DEC_MAXB][PAY / 16];
    uint16_t dwh[DEC_MAXB];
#pragma unroll
    for (int j = 0; j < DEC_MAXB; j++) {
        if (b0 + j < b1) {
            const uint4* src = (const uint4*)(wp + (int64_t)(b0 + j) * 64 * PAY);
#pragma unroll
            for (int c = 0; c < PAY / 16; c++) wv[j][c] = src[c];
            dwh[j] = ws[(int64_t)(b0 + j) * 64];
        }
    }
    // ---- per-block terms of every assignment (unrolled: the rows stay in scalar registers)
#pragma unroll
    for (int i = 0; i < DEC_A; i++) {
        if (i >= cnt) break;
        const int64_t r = arow[i];
        const uint32_t* xq = (const uint32_t*)(M.in.q + r * M.in.qstride);
        const float* xd = M.in.d + r * M.in.dstride;
        const int* xs = M.in.s + r * M.in.sstride;
#pragma unroll
        for (int j = 0; j < DEC_MAXB; j++) {
            const int b = b0 + j;
            if (b < b1) {
                const uint32_t* xb = xq + b * 8;
                int isum = 0;
                if (TYPE == PHX_Q4_0_DEV) {
                    const uint32_t w4[4] = {wv[j][0].x, wv[j][0].y, wv[j][0].z, wv[j][0].w};
#pragma unroll
                    for (int w = 0; w < 4; w++) {
                        isum = __builtin_amdgcn_sdot4((int)(w4[w] & 0x0F0F0F0Fu), (int)xb[w], isum, false);
                        isum = __builtin_amdgcn_sdot4((int)((w4[w] >> 4) & 0x0F0F0F0Fu), (int)xb[4 + w], isum, false);
                    }
                    isum -= 8 * xs[b];
                } else {
                    const uint32_t w8[8] = {wv[j][0].x, wv[j][0].y, wv[j][0].z, wv[j][0].w,
                                            wv[j][PAY / 16 - 1].x, wv[j][PAY / 16 - 1].y, wv[j][PAY / 16 - 1].z,
                                            wv[j][PAY / 16 - 1].w};
#pragma unroll
                    for (int w = 0; w < 8; w++) isum = __builtin_amdgcn_sdot4((int)w8[w], (int)xb[w], isum, false);
                }
                const float dd = h2f(dwh[j]) * xd[b];
                terms[i][b][lane] = (float)isum * dd;
            }
        }
    }
    __syncthreads();
    // ---- the float chain in block order (wave i for assignment i), then the epilogue
    if (wave < cnt) {
        const int i = wave;
        float S = 0.0f;
#pragma unroll 8
        for (int b = 0; b < nb; b++) S += terms[i][b][lane];
        const int64_t orr = orow[i];
        if (MODE == 0) {
            // paired row group: lanes 0-31 gate j, lanes 32-63 up j, j = 32 rgi + lane % 32
            const int jj = rgi * 32 + (lane & 31);
            const float u = __shfl_down(S, 32, 64);
            if (jj < M.split) {
                if (lane < 32) M.out0[orr * M.split + jj] = S;
                else M.out1[orr * M.split + jj] = S;
            }
            const float ev = lane < 32 ? gelu_ref(S, a.gelu_tab) * u : 0.0f;
            float dval;
            int sum;
            const int q = q8_0_half(ev, &dval, &sum);
            if (lane < 32) {
                const Act& o = M.out_act;
                o.q[orr * o.qstride + jj] = (int8_t)q;
                if (lane == 0) {
                    o.d[orr * o.dstride + rgi] = dval;
                    o.s[orr * o.sstride + rgi] = sum;
                }
            }
        } else {
            const int row = rgi * 64 + lane;
            if (row < M.rows) M.out0[orr * M.rows + row] = S;
        }
    }
}

static DecMat to_dev(const DecMatH& h)
{
    DecMat m{};
    if (!h.q) return m;
    m.pay = h.q->payload;
    m.sc = h.q->scale;
    m.mat_pay = h.q->mat_pay_stride();
    m.mat_sc = h.q->mat_sc_stride();
    m.rg = h.q->rg;
    m.nb = h.q->nb;
    m.rows = h.q->rows;
    m.in = h.in;
    m.out0 = h.out0;
    m.out1 = h.out1;
    m.split = h.split;
    m.out_act = h.out_act;
    return m;
}

void launch_dec(hipStream_t st, int mode, const DecMatH& m0, const DecMatH& m1, const DecTile* tiles, int max_tiles,
                int act_div, int T, const float* gelu_tab)
{
    DecArgs a{};
    a.m0 = to_dev(m0);
    a.m1 = to_dev(m1);
    a.tiles = tiles;
    a.max_tiles = max_tiles;
    a.act_div = act_div;
    a.T = T;
    a.gelu_tab = gelu_tab;
    const int items = max_tiles * a.m0.rg + (a.m1.rg > 0 ? (T + DEC_A - 1) / DEC_A * a.m1.rg : 0);
    const bool q4 = m0.q->type == PHX_Q4_0_DEV;
    // 8 waves share a row's blocks (nb <= 128)
    if (mode == 0) {
        if (q4) launch((k_dec_mm<0, PHX_Q4_0_DEV, 8, 16>), dim3(items), dim3(512), 0, st, a);
        else launch((k_dec_mm<0, PHX_Q8_0_DEV, 8, 16>), dim3(items), dim3(512), 0, st, a);
    } else {
        if (q4) launch((k_dec_mm<1, PHX_Q4_0_DEV, 8, 16>), dim3(items), dim3(512), 0, st, a);
        else launch((k_dec_mm<1, PHX_Q8_0_DEV, 8, 16>), dim3(items), dim3(512), 0, st, a);
    }
}

// ------------------------------------------------------------------------------ combine (decode)
// k_combine's arithmetic (rank-ordered sum of w_j * yd_j, the two branch norms, optional residual;
// src/GemmaCpu.cs:384,418-421,355-356) with 1024 threads per token and every global load of the
// token issued in one round (d <= 4096, k <= 16).
constexpr int CB_NT = 1024, CB_MAXE = 4;

__global__ __launch_bounds__(CB_NT) void k_combine_dec(int d, int k, float eps, const float* __restrict__ yd,
                                                       const float* __restrict__ w, const float* __restrict__ shared,
                                                       const float* __restrict__ post1, const float* __restrict__ post2,
                                                       float* __restrict__ out, float* __restrict__ xres,
                                                       const float* __restrict__ post_ffw, int* flags)
{
    extern __shared__ float cb[];  // acc [d], shared [d], out [d]
    __shared__ double red[CB_NT / 64 + 1];
    const int t = blockIdx.x, tid = threadIdx.x;
    float* sacc = cb;
    float* ssh = cb + d;
    float* so = cb + 2 * d;
    const float* sh = shared ? shared + (int64_t)t * d : nullptr;
    float wj[PHX_MAX_USED_DEV];
#pragma unroll
    for (int j = 0; j < PHX_MAX_USED_DEV; j++) wj[j] = j < k ? w[(int64_t)t * k + j] : 0.0f;
    float yv[CB_MAXE][PHX_MAX_USED_DEV], shv[CB_MAXE], p1[CB_MAXE], p2[CB_MAXE], pf[CB_MAXE], xv[CB_MAXE];
#pragma unroll
    for (int q = 0; q < CB_MAXE; q++) {
        const int i = tid + q * CB_NT;
        const bool in = i < d;
#pragma unroll
        for (int j = 0; j < PHX_MAX_USED_DEV; j++) yv[q][j] = (in && j < k) ? yd[((int64_t)t * k + j) * d + i] : 0.0f;
        shv[q] = (in && sh) ? sh[i] : 0.0f;
        p1[q] = (in && sh) ? post1[i] : 0.0f;
        p2[q] = in ? post2[i] : 0.0f;
        pf[q] = (in && xres) ? post_ffw[i] : 0.0f;
        xv[q] = (in && xres) ? xres[(int64_t)t * d + i] : 0.0f;
    }
    float accv[CB_MAXE];
#pragma unroll
    for (int q = 0; q < CB_MAXE; q++) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < PHX_MAX_USED_DEV; j++)
            if (j < k) acc += yv[q][j] * wj[j];
        accv[q] = acc;
        const int i = tid + q * CB_NT;
        if (i < d) {
            sacc[i] = acc;
            ssh[i] = shv[q];
        }
    }
    __syncthreads();
    const float s2 = rms_scale_from_mean(mean_sq_cert<CB_NT>(sacc, d, red, flags), eps);
    const float s1 = sh ? rms_scale_from_mean(mean_sq_cert<CB_NT>(ssh, d, red, flags), eps) : 0.0f;
    float ov[CB_MAXE];
#pragma unroll
    for (int q = 0; q < CB_MAXE; q++) {
        const int i = tid + q * CB_NT;
        const float mlp = sh ? shv[q] * s1 * p1[q] : 0.0f;
        ov[q] = mlp + accv[q] * s2 * p2[q];
        if (i < d) {
            out[(int64_t)t * d + i] = ov[q];
            so[i] = ov[q];
        }
    }
    if (xres) {
        __syncthreads();
        const float s3 = rms_scale_from_mean(mean_sq_cert<CB_NT>(so, d, red, flags), eps);
#pragma unroll
        for (int q = 0; q < CB_MAXE; q++) {
            const int i = tid + q * CB_NT;
            if (i < d) xres[(int64_t)t * d + i] = xv[q] + ov[q] * s3 * pf[q];
        }
    }
}

void launch_combine_dec(hipStream_t st, int T, int d, int k, float eps, const float* yd, const float* w,
                        const float* shared, const float* post1, const float* post2, float* out, float* xres,
                        const float* post_ffw, int* flags)
{
    launch(k_combine_dec, dim3(T), dim3(CB_NT), (size_t)3 * d * sizeof(float), st, d, k, eps, yd, w, shared,
                       post1, post2, out, xres, post_ffw, flags);
}

}  // namespace phx
