// Device helpers shared by the kernels: exact conversions and roundings of the reference CPU path,
// wave reductions, and the certified double-precision mean of squares of RmsNorm.
#pragma once
#include <hip/hip_fp16.h>

#include <type_traits>

#include "phx_internal.h"

namespace phx {

// Clock stamps of kernel phases, compiled only into an instrumented build (-DPHX_TIMELINE; one table
// per source file): thread 0 of
// workgroup b (< TL_WG) writes the 100 MHz wall clock at phase `slot` of launch kind `kind` of stack
// layer `seq` (modulo TL_SEQ); phxdbg_timeline copies the table to the host.  Without the macro the
// stamps compile to nothing.
#ifdef PHX_TIMELINE
constexpr int TL_SEQ = 64, TL_KIND = 4, TL_SLOT = 12, TL_WG = 512;
static __device__ unsigned long long phx_tl[TL_SEQ * TL_KIND * TL_SLOT * TL_WG];
#define TL_STAMP(seq, kind, slot)                                                                   \
    do {                                                                                            \
        if (threadIdx.x == 0 && blockIdx.x < TL_WG)                                                 \
            phx_tl[((((seq) % TL_SEQ) * TL_KIND + (kind)) * TL_SLOT + (slot)) * TL_WG + blockIdx.x] = \
                wall_clock64();                                                                     \
    } while (0)
// the workgroup's compute unit instead of a time: XCC_ID << 16 | HW_ID bits 8-15 (CU, SH, SE)
#define TL_HWID(seq, kind, slot)                                                                          \
    do {                                                                                                  \
        if (threadIdx.x == 0 && blockIdx.x < TL_WG)                                                       \
            phx_tl[((((seq) % TL_SEQ) * TL_KIND + (kind)) * TL_SLOT + (slot)) * TL_WG + blockIdx.x] =       \
                ((unsigned long long)(__builtin_amdgcn_s_getreg((31 << 11) | 20) & 0xF) << 16) |           \
                ((__builtin_amdgcn_s_getreg((31 << 11) | 4) >> 8) & 0xFF) | (1ull << 62);                  \
    } while (0)
// the stamp once the wave's outstanding loads have landed (the wait itself only in the instrumented build)
#define TL_STAMP_LANDED(seq, kind, slot)  \
    do {                                  \
        __builtin_amdgcn_s_waitcnt(0);    \
        TL_STAMP(seq, kind, slot);        \
    } while (0)
#else
#define TL_STAMP(seq, kind, slot) ((void)0)
#define TL_STAMP_LANDED(seq, kind, slot) ((void)0)
#define TL_HWID(seq, kind, slot) ((void)0)
#endif

// ------------------------------------------------------------------------------ scalar helpers

// fp16 bits -> float (exact: every binary16 value is a binary32 value; f16 denormals are kept)
__device__ __forceinline__ float h2f(uint32_t h) { return __half2float(__ushort_as_half((unsigned short)h)); }

// float -> fp16 bits, round to nearest even with subnormals: the rounding rule of Half.FromFloat
// (src/Half.cs:26-54), which is IEEE binary16 conversion except that every NaN becomes the quiet NaN
// sign | 0x7E00.  The hardware conversion (round to nearest even; fp16 denormals are not flushed in
// the default mode) gives the same bits for every non-NaN value; the NaN case is fixed up here.
__device__ __forceinline__ uint32_t f2h_bits(float value)
{
    const uint32_t h = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)value);
    return value != value ? (h & 0x8000u) | 0x7E00u : h;
}

// C's nearest_int through 1.5*2^23 (src/CpuRefKQuants.cs:45-51)
__device__ __forceinline__ int nearest_int(float f)
{
    float val = f + 12582912.0f;
    int i = __float_as_int(val);
    return (i & 0x007fffff) - 0x00400000;
}

// 1f / (float)sqrt((double)(mean + eps)), the scale expression of CpuRef.RmsNorm (src/CpuRef.cs:188-189)
__device__ __forceinline__ float rms_scale_from_mean(float mean, float eps)
{
    float me = mean + eps;
    return 1.0f / (float)__dsqrt_rn((double)me);
}

// GELU of the reference (src/CpuRefGemma.cs:85-92): 0 at or below -10, x at or above 10, otherwise
// a function of fp16(x) only, read from the 65,536-entry table the runtime builds at context creation.
__device__ __forceinline__ float gelu_ref(float x, const float* __restrict__ tab)
{
    if (x <= -10.0f) return 0.0f;
    if (x >= 10.0f) return x;
    return tab[f2h_bits(x)];
}

// (key, index) pair `o` beats `b`: higher key, or equal key and lower index; index < 0 is empty.
// Keys compared with it are never NaN.
template <class F>
__device__ __forceinline__ bool sel_beats(F ov, int oi, F bv, int bi)
{
    return oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi));
}

// Top-k rounds of the reference (src/GemmaCpu.cs:400-405): a round starts from the lowest-index
// untaken expert e0 and replaces the current one only by a strictly greater logit.  Nothing compares
// greater than NaN and NaN compares greater than nothing, so a round takes e0 when its logit is NaN,
// and otherwise the largest non-NaN logit among the untaken experts, the lower index on ties.
// scan_start finds e0 over a wave holding expert lane + 64 q in slot q: its index (-1 when no expert
// is left, in every lane) and whether its logit is NaN.
template <class F>
__device__ __forceinline__ int scan_start(const bool (&avail)[4], const F (&v)[4], bool* e0_nan)
{
    int e0 = -1;
    bool nan0 = false;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const uint64_t m = __ballot(avail[q]);
        const uint64_t n = __ballot(avail[q] && v[q] != v[q]);
        if (e0 < 0 && m != 0ull) {
            const int l = __builtin_ctzll(m);
            e0 = 64 * q + l;
            nan0 = (n >> l) & 1ull;
        }
    }
    *e0_nan = nan0;
    return e0;
}

// An expert id outside [0, E) can only come from a bug upstream; it is mapped into range so no list
// write leaves its buffer.
__device__ __forceinline__ int clamp_id(int e, int E) { return e < 0 ? 0 : (e >= E ? E - 1 : e); }

// ---- DPP reductions (VALU-latency lane exchanges; gfx9 row_bcast for the cross-row steps)
template <int CTRL, int ROWMASK = 0xf>
__device__ __forceinline__ int dpp_i(int old, int v)
{
    return __builtin_amdgcn_update_dpp(old, v, CTRL, ROWMASK, 0xf, false);
}
template <int CTRL, int ROWMASK = 0xf>
__device__ __forceinline__ float dpp_f(float old, float v)
{
    return __int_as_float(dpp_i<CTRL, ROWMASK>(__float_as_int(old), __float_as_int(v)));
}
template <int CTRL, int ROWMASK = 0xf>
__device__ __forceinline__ double dpp_d(double old, double v)
{
    const long long o = __double_as_longlong(old), x = __double_as_longlong(v);
    const int lo = dpp_i<CTRL, ROWMASK>((int)o, (int)x);
    const int hi = dpp_i<CTRL, ROWMASK>((int)(o >> 32), (int)(x >> 32));
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

// Sum of a 16-lane row, in every lane of the row (quad swaps, half mirror, mirror).
template <class F>
__device__ __forceinline__ F row_sum(F v)
{
    if constexpr (sizeof(F) == 8) {
        v += dpp_d<0xb1>(0.0, v);
        v += dpp_d<0x4e>(0.0, v);
        v += dpp_d<0x141>(0.0, v);
        v += dpp_d<0x140>(0.0, v);
    } else if constexpr (std::is_same<F, float>::value) {
        v += dpp_f<0xb1>(0.0f, v);
        v += dpp_f<0x4e>(0.0f, v);
        v += dpp_f<0x141>(0.0f, v);
        v += dpp_f<0x140>(0.0f, v);
    } else {
        v += dpp_i<0xb1>(0, v);
        v += dpp_i<0x4e>(0, v);
        v += dpp_i<0x141>(0, v);
        v += dpp_i<0x140>(0, v);
    }
    return v;
}

__device__ __forceinline__ float row_max(float v)
{
    v = fmaxf(v, dpp_f<0xb1>(v, v));
    v = fmaxf(v, dpp_f<0x4e>(v, v));
    v = fmaxf(v, dpp_f<0x141>(v, v));
    v = fmaxf(v, dpp_f<0x140>(v, v));
    return v;
}

// Sum over the 64 lanes, the same value returned to every lane: rows are summed, rows 0+1 and 2+3
// combined through row_bcast15, then row_bcast31; lane 63 holds the total.
__device__ __forceinline__ double wave_sum_dpp(double v)
{
    v = row_sum(v);
    v += dpp_d<0x142, 0xa>(0.0, v);
    v += dpp_d<0x143, 0xc>(0.0, v);
    const long long t = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)t, 63), hi = __builtin_amdgcn_readlane((int)(t >> 32), 63);
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

// Float sum over the 64 lanes (the same tree as wave_sum_dpp), returned to every lane.
__device__ __forceinline__ float wave_sum_f(float v)
{
    v = row_sum(v);
    v += dpp_f<0x142, 0xa>(0.0f, v);
    v += dpp_f<0x143, 0xc>(0.0f, v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Sum / max over each 32-lane half (lanes 0-31 and 32-63), returned to the lanes of that half.
__device__ __forceinline__ int half_sum_i(int v)
{
    v = row_sum(v);
    v += dpp_i<0x142, 0xa>(0, v);
    const int a = __builtin_amdgcn_readlane(v, 31), b = __builtin_amdgcn_readlane(v, 63);
    return (threadIdx.x & 32) ? b : a;
}

__device__ __forceinline__ float half_max_f(float v)
{
    v = row_max(v);
    v = fmaxf(v, dpp_f<0x142, 0xa>(v, v));
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
    return (threadIdx.x & 32) ? b : a;
}

// Q8_0 of 32 values held one per lane of a 32-lane half (CpuRef.QuantizeQ8_0, src/CpuRef.cs:49-62):
// returns q; *dval the block scale as its fp16 value, *sum the block's integer sum.
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

typedef _Float16 mh2 __attribute__((ext_vector_type(2)));

// Bytes to exact fp16 pairs by the 1024-bias: the half with bits 0x64XX is 1024 + XX.  Returns the
// pair (byte 2p, byte 2p + 1) of w minus `bias` (1152 gives a signed int8 from w ^ 0x80808080,
// 1032 gives q - 8 from a nibble).
__device__ __forceinline__ uint32_t bias_pair(uint32_t w, int p, float bias)
{
    const uint32_t b = __builtin_amdgcn_perm(0x64646464u, w, p ? 0x04030402u : 0x04010400u);
    mh2 v = __builtin_bit_cast(mh2, b);
    v = v - mh2{(_Float16)bias, (_Float16)bias};
    return __builtin_bit_cast(uint32_t, v);
}

// Four Q8_0 integers (bytes of qw) as fp16 halves: exact (signed bytes through the 1152 bias), or, for
// the tolerance mode's operands, times the block scale d (an fp16 value: q * d is exact in float) and
// rounded once to fp16.
__device__ __forceinline__ uint2 int_q4(int qw)
{
    const uint32_t u = (uint32_t)qw ^ 0x80808080u;
    return make_uint2(bias_pair(u, 0, 1152.0f), bias_pair(u, 1, 1152.0f));
}
__device__ __forceinline__ uint32_t fold_pair(int q0, int q1, float d)
{
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)((float)q0 * d)) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)((float)q1 * d)) << 16);
}
__device__ __forceinline__ uint2 fold_q4(int qw, float d)
{
    return make_uint2(fold_pair((int8_t)(qw & 0xFF), (int8_t)((qw >> 8) & 0xFF), d),
                      fold_pair((int8_t)((qw >> 16) & 0xFF), (int8_t)(qw >> 24), d));
}

// Q8_0 of one 32-block held as 4 consecutive values per lane by an 8-lane group (lane l of the group:
// elements 4l..4l+3), CpuRef.QuantizeQ8_0 (src/CpuRef.cs:49-62): amax, d = amax / 127, id = 1 / d,
// q = roundf(x * id) (half away from zero), fp16 d.  Returns the lane's 4 q bytes as one dword (the
// LDS activation layout); *dval and *sum (the block's q sum) are valid in all 8 lanes.
__device__ __forceinline__ int q8_0_oct(float4 v, float* dval, int* sum)
{
    // the 8-lane maximum and sum by DPP (quad swaps, then the other quad through the half-row mirror);
    // both are exact in any order
    float am = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
    am = fmaxf(am, dpp_f<0xb1>(am, am));
    am = fmaxf(am, dpp_f<0x4e>(am, am));
    am = fmaxf(am, dpp_f<0x141>(am, am));
    const float dd = am / 127.0f;
    const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
    const int q0 = (int)roundf(v.x * id), q1 = (int)roundf(v.y * id), q2 = (int)roundf(v.z * id),
              q3 = (int)roundf(v.w * id);
    int sm = q0 + q1 + q2 + q3;
    sm += dpp_i<0xb1>(sm, sm);
    sm += dpp_i<0x4e>(sm, sm);
    sm += dpp_i<0x141>(sm, sm);
    *dval = h2f(f2h_bits(dd));
    *sum = sm;
    return (q0 & 0xFF) | ((q1 & 0xFF) << 8) | ((q2 & 0xFF) << 16) | (int)((unsigned)q3 << 24);
}


// Maximum over the 64 lanes of an unsigned 64-bit key (returned to every lane).
__device__ __forceinline__ bool u64_gt(unsigned hi_a, unsigned lo_a, unsigned hi_b, unsigned lo_b)
{
    return hi_a > hi_b || (hi_a == hi_b && lo_a > lo_b);
}
template <int CTRL, int ROWMASK = 0xf>
__device__ __forceinline__ void u64_max_step(unsigned& hi, unsigned& lo)
{
    const unsigned ohi = (unsigned)dpp_i<CTRL, ROWMASK>((int)hi, (int)hi);
    const unsigned olo = (unsigned)dpp_i<CTRL, ROWMASK>((int)lo, (int)lo);
    if (u64_gt(ohi, olo, hi, lo)) { hi = ohi; lo = olo; }
}
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long v)
{
    unsigned hi = (unsigned)(v >> 32), lo = (unsigned)v;
    u64_max_step<0xb1>(hi, lo);
    u64_max_step<0x4e>(hi, lo);
    u64_max_step<0x141>(hi, lo);
    u64_max_step<0x140>(hi, lo);
    u64_max_step<0x142, 0xa>(hi, lo);
    u64_max_step<0x143, 0xc>(hi, lo);
    hi = (unsigned)__builtin_amdgcn_readlane((int)hi, 63);
    lo = (unsigned)__builtin_amdgcn_readlane((int)lo, 63);
    return ((unsigned long long)hi << 32) | lo;
}

// Maximum over the 64 lanes of an unsigned 32-bit value, returned to every lane: six in-place maxima
// with a DPP operand (quad swaps, half mirror, mirror, then the row broadcasts into rows 1, 3 and
// 2, 3); the compiler would copy the value through a separate DPP move at every step.  Each step reads
// the previous step's result through DPP, two wait states after it is written.
__device__ __forceinline__ unsigned wave_max_u32(unsigned v)
{
    asm volatile(
        "s_nop 1\n\t"
        "v_max_u32_dpp %0, %0, %0 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_max_u32_dpp %0, %0, %0 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_max_u32_dpp %0, %0, %0 row_half_mirror row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_max_u32_dpp %0, %0, %0 row_mirror row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_max_u32_dpp %0, %0, %0 row_bcast:15 row_mask:0xa bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_max_u32_dpp %0, %0, %0 row_bcast:31 row_mask:0xc bank_mask:0xf\n\t"
        "s_nop 1"
        : "+v"(v));
    return (unsigned)__builtin_amdgcn_readlane((int)v, 63);
}

// Maximum over the 64 lanes of the 64-bit key (hi, lo), returned to every lane.
template <int CTRL, int ROWMASK = 0xf>
__device__ __forceinline__ void key_max_step(unsigned& hi, unsigned& lo)
{
    const unsigned oh = (unsigned)dpp_i<CTRL, ROWMASK>((int)hi, (int)hi), ol = (unsigned)dpp_i<CTRL, ROWMASK>((int)lo, (int)lo);
    const bool gt = oh > hi || (oh == hi && ol > lo);
    hi = gt ? oh : hi;
    lo = gt ? ol : lo;
}
__device__ __forceinline__ void wave_max_key(unsigned& hi, unsigned& lo)
{
    key_max_step<0xb1>(hi, lo);
    key_max_step<0x4e>(hi, lo);
    key_max_step<0x141>(hi, lo);
    key_max_step<0x140>(hi, lo);
    key_max_step<0x142, 0xa>(hi, lo);
    key_max_step<0x143, 0xc>(hi, lo);
    hi = (unsigned)__builtin_amdgcn_readlane((int)hi, 63);
    lo = (unsigned)__builtin_amdgcn_readlane((int)lo, 63);
}

// Maximum over the 64 lanes of a double (NaN-free inputs), returned to every lane.
__device__ __forceinline__ double wave_max_dpp(double v)
{
    v = fmax(v, dpp_d<0xb1>(v, v));
    v = fmax(v, dpp_d<0x4e>(v, v));
    v = fmax(v, dpp_d<0x141>(v, v));
    v = fmax(v, dpp_d<0x140>(v, v));
    v = fmax(v, dpp_d<0x142, 0xa>(v, v));
    v = fmax(v, dpp_d<0x143, 0xc>(v, v));
    const long long t = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)t, 63), hi = __builtin_amdgcn_readlane((int)(t >> 32), 63);
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

// Inclusive prefix sum of an int over the 64 lanes (the same steps as the double one below).
__device__ __forceinline__ int wave_incl_scan_i(int v)
{
    v += dpp_i<0x111>(0, v);  // row_shr:1
    v += dpp_i<0x112>(0, v);  // row_shr:2
    v += dpp_i<0x114>(0, v);  // row_shr:4
    v += dpp_i<0x118>(0, v);  // row_shr:8
    v += dpp_i<0x142, 0xa>(0, v);  // row_bcast:15 into rows 1 and 3
    v += dpp_i<0x143, 0xc>(0, v);  // row_bcast:31 into rows 2 and 3
    return v;
}

// Inclusive prefix sum over the 64 lanes (row shifts within 16-lane rows, then row broadcasts).
__device__ __forceinline__ double wave_incl_scan_dpp(double v)
{
    v += dpp_d<0x111>(0.0, v);  // row_shr:1
    v += dpp_d<0x112>(0.0, v);  // row_shr:2
    v += dpp_d<0x114>(0.0, v);  // row_shr:4
    v += dpp_d<0x118>(0.0, v);  // row_shr:8
    v += dpp_d<0x142, 0xa>(0.0, v);  // row_bcast:15 into rows 1 and 3
    v += dpp_d<0x143, 0xc>(0.0, v);  // row_bcast:31 into rows 2 and 3
    return v;
}

// Order-preserving map of a float to uint32 (NaN to 0, below every number; the certified selection
// never accepts an order with a NaN logit, see wave_topk).
__device__ __forceinline__ unsigned sortable_f32(float f)
{
    if (f != f) return 0u;
    const unsigned b = __float_as_uint(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// The two float ends of (S -/+ B) / n, the interval of means a certified sum of squares S (error bound
// B, S >= 0) allows, formed with the reciprocal rn = 1 / n instead of a double division: the bound is
// widened by S * 2^-49, above the relative error of rn and of the product (under 2^-51), so the ends
// still bracket the reference's (double)(sum / n) for every sum in [S - B, S + B]; equal ends are the
// reference's (float)(sum / n) (division and both roundings are monotone).
__device__ __forceinline__ void mean_ends(double S, double B, double rn, float* lo, float* hi)
{
    const double Bw = B + S * 0x1p-49;
    *lo = (float)((S - Bw) * rn);
    *hi = (float)((S + Bw) * rn);
}

// ------------------------------------------------------------------------------ sequential sum of squares
// The reference's sum of squares q = ((0 + x_0^2) + x_1^2) + ... + x_{n-1}^2 in double, in index order
// (CpuRef.RmsNorm, src/CpuRef.cs:186-187), bit for bit, by one wave (all 64 lanes, uniform control flow)
// with far fewer than n dependent additions.  Every x_i^2 is exact in double and every partial sum is
// >= 0, so the chain only climbs.  While it stays in one binade [2^e, 2^(e+1)) its values are multiples
// of g = 2^(e-52) and each step adds x_i^2 rounded to a multiple of g: to nearest, and at an exact half
// to the even multiple of the sum, so the step count of g is fixed by x_i and the parity of the sum
// before it (and the sum is even right after such a step).  Lane c takes the chunk [c C, (c + 1) C),
// C = ceil(n / 64), and counts its steps for either starting parity when the chunk lies in one binade:
// the chain stays within (n + 128) 2^-51 of the exact prefix sums, and the wave's scan of the chunk sums
// within that of them too, so the chunk's ends bound it.  A walk over the 64 chunks then adds each such
// chunk's count for the parity the sum has at its start and replays the others (the first chunk, those
// where the sum crosses a power of two: about 7 of 64 for rows of like terms, non-finite ones) term by
// term.  Short rows are summed term by term.
__device__ __forceinline__ double seq_sum_sq_serial(const float* x, int b, int e, double q)
{
    int i = b;
    for (; i + 8 <= e; i += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = x[i + j];
#pragma unroll
        for (int j = 0; j < 8; j++) q = fma((double)v[j], (double)v[j], q);  // x^2 exact: one rounding
    }
    for (; i < e; i++) q = fma((double)x[i], (double)x[i], q);
    return q;
}

// a wave-uniform double from lane c (c uniform)
__device__ __forceinline__ double readlane_d(double v, int c)
{
    const long long t = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)t, c), hi = __builtin_amdgcn_readlane((int)(t >> 32), c);
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

// whether the integer-valued double v (0 <= v < 2^53) is odd
__device__ __forceinline__ bool odd_d(double v) { return floor(v * 0.5) != v * 0.5; }

__device__ __noinline__ double seq_sum_sq_wave(const float* x, int n)
{
    if (n < 512) return seq_sum_sq_serial(x, 0, n, 0.0);
    const int lane = threadIdx.x & 63, C = (n + 63) / 64;
    const int b = min(n, lane * C), e = min(n, b + C);
    double Q = 0.0;
    for (int i = b; i < e; i++) Q = fma((double)x[i], (double)x[i], Q);
    double inc = Q;  // inclusive scan of the chunk sums, then the exclusive one: A = the chunks before
#pragma unroll
    for (int k = 1; k < 64; k *= 2) {
        const double y = __shfl_up(inc, k, 64);
        if (lane >= k) inc += y;
    }
    double A = __shfl_up(inc, 1, 64);
    if (lane == 0) A = 0.0;
    const double eps = ((double)n + 128.0) * 0x1p-50;  // twice the chain's and the scan's relative error
    const double lo = A * (1.0 - eps), hi = (A + Q) * (1.0 + eps);
    int el = 0, eh = 1;
    if (lo > 0.0 && hi < INFINITY) {
        frexp(lo, &el);
        frexp(hi, &eh);
    }
    const int ex = el - 1;  // lo in [2^ex, 2^(ex + 1))
    // the chunk's count of g = 2^(ex - 52) for a start of even parity (d0), and the odd start's difference
    // at its first half-way term (after it both sums are even and agree)
    double d0 = 0.0;
    int diff = 0, ties = 0;
    const bool clean = b < e && el == eh;
    if (clean) {
        for (int i = b; i < e; i++) {
            const double t = (double)x[i] * (double)x[i];
            const double v = ldexp(t, 52 - ex), fl = floor(v), f = v - fl;
            double step = f > 0.5 ? fl + 1.0 : fl;
            if (f == 0.5) {  // to the even multiple: (start + d0 + fl) even keeps fl, else fl + 1
                const bool up = odd_d(d0) != odd_d(fl);  // even start
                step = up ? fl + 1.0 : fl;
                if (ties++ == 0) diff = up ? -1 : 1;  // the odd start rounds the other way
            }
            d0 += step;
        }
    }
    // the walk: each clean chunk's count for the parity of the sum at its start, the others term by term
    const int info = clean ? ((ex + 2048) << 2 | (ties ? 2 : 0) | 1) : 0;
    double q = 0.0;
    for (int c = 0; c < 64; c++) {  // uniform
        const int cb = min(n, c * C), ce = min(n, cb + C);
        if (cb >= ce) break;
        const int ci = __builtin_amdgcn_readlane(info, c);
        if (ci & 1) {
            const int cx = (ci >> 2) - 2048;
            double D = readlane_d(d0, c);
            // q lies in [2^cx, 2^(cx + 1)): its last significand bit is its parity in g
            if ((ci & 2) && (__double_as_longlong(q) & 1)) D += (double)__builtin_amdgcn_readlane(diff, c);
            q += ldexp(D, cx - 52);  // exact: the result is the chain's value
        } else {
            q = seq_sum_sq_serial(x, cb, ce, q);
        }
    }
    return q;
}

// Mean of squares of one row as CpuRef.RmsNorm rounds it: (float)(sum / n) with sum the double sum of
// x_i^2 in index order (src/CpuRef.cs:186-188).  A parallel double sum differs from the sequential
// one by at most (n + per + depth) * 2^-53 * sum (all terms are non-negative); when both ends of
// that interval give the same float the result is certain, otherwise one thread re-sums
// sequentially (rare; counted in fallbacks[0]).  Block-level: NT threads, red >= NT/64 + 1 doubles.
template <int NT>
__device__ float mean_sq_cert_from(double s, int per, const float* x, int n, double* red, int* fallbacks);

template <int NT>
__device__ float mean_sq_cert(const float* x, int n, double* red, int* fallbacks)
{
    const int tid = threadIdx.x;
    double s = 0.0;
    for (int i = tid; i < n; i += NT) {
        double v = (double)x[i];
        s += v * v;
    }
    return mean_sq_cert_from<NT>(s, (n + NT - 1) / NT, x, n, red, fallbacks);
}

// The same from each thread's own double sum s of at most `per` squares (any partition of the row):
// the wave and workgroup sums, the bound and, if it cannot certify the rounding, the sequential sum.
template <int NT>
__device__ float mean_sq_cert_from(double s, int per, const float* x, int n, double* red, int* fallbacks)
{
    constexpr int NW = NT / 64;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    s = wave_sum_dpp(s);
    if (lane == 0) red[wave] = s;
    __syncthreads();
    double S = 0.0;
    for (int w = 0; w < NW; w++) S += red[w];
    const double B = ((double)n + per + 64.0) * 0x1p-53 * S * 2.0;
    float lo, hi;
    mean_ends(S, B, 1.0 / (double)n, &lo, &hi);
    float mean = lo;
    if (lo != hi) {
        __syncthreads();
        if (tid < 64) {
            const double q = seq_sum_sq_wave(x, n);
            if (tid == 0) {
                red[NW] = q;
                if (fallbacks) atomicAdd(fallbacks, 1);
            }
        }
        __syncthreads();
        mean = (float)(red[NW] / (double)n);
    }
    __syncthreads();
    return mean;
}

// ------------------------------------------------------------------------------ explicit LDS reads
// Kernels that fill LDS with direct global -> LDS loads read it back with these: the compiler would
// otherwise wait for every outstanding direct load before any LDS read it emits.
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void* lds_void_t;
typedef __attribute__((address_space(1))) void* glb_void_t;

// explicit LDS reads at address a + OFF (asynchronous: the value is valid after lds_wait)
template <int OFF = 0>
__device__ __forceinline__ u32x4 ds_r128(uint32_t a)
{
    u32x4 v;
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(a), "i"(OFF));
    return v;
}
template <int OFF = 0>
__device__ __forceinline__ u32x2 ds_r64(uint32_t a)
{
    u32x2 v;
    asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(v) : "v"(a), "i"(OFF));
    return v;
}
template <int OFF = 0>
__device__ __forceinline__ uint32_t ds_r32(uint32_t a)
{
    uint32_t v;
    asm volatile("ds_read_b32 %0, %1 offset:%2" : "=v"(v) : "v"(a), "i"(OFF));
    return v;
}
template <int OFF = 0>
__device__ __forceinline__ uint32_t ds_ru16(uint32_t a)
{
    uint32_t v;
    asm volatile("ds_read_u16 %0, %1 offset:%2" : "=v"(v) : "v"(a), "i"(OFF));
    return v;
}

// A raw buffer resource (gfx9 descriptor, stride 0) over the 4 GB from p: a direct buffer -> LDS load
// through it takes its lane offset from a VGPR and a uniform offset from an SGPR, so a loop that walks
// a row advances a scalar instead of each lane's 64-bit address.  The range covers every 32-bit
// offset; no access relies on the range check.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void* p)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, -1, 0x00020000);
}
// waits for every LDS read of the wave; the registers passed are the reads' results, tied to the wait
// so that no use of them is scheduled above it.  A read's result must have no other use before its
// wait, and the read and its wait must sit in one basic block: the compiler takes an asm result as
// ready at once, so a copy it placed in between (to split a value, or at a branch join) would copy
// the register before the data lands.
__device__ __forceinline__ void lds_wait(u32x4& a, u32x4& b, uint32_t& c)
{
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c)::"memory");
}
__device__ __forceinline__ void lds_wait(u32x4& a, u32x4& b, uint32_t& c, u32x2& d, uint32_t& f)
{
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d), "+v"(f)::"memory");
}
__device__ __forceinline__ void lds_wait(u32x4& a, u32x4& b, uint32_t& c, u32x2& d, u32x2& e, uint32_t& f)
{
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a), "+v"(b), "+v"(c), "+v"(d), "+v"(e), "+v"(f)::"memory");
}
// s_waitcnt vmcnt(n) alone (gfx9 encoding: vmcnt bits 3:0 and 15:14)
constexpr int vm_wait(int n) { return (n & 15) | ((n >> 4) << 14) | (0x7 << 4) | (0xF << 8); }
// compile-time index for unrolled steps with immediate offsets
template <int N> using ic = std::integral_constant<int, N>;
// f(ic<0>), f(ic<1>), ..., f(ic<N - 1>) in order
template <int N, int I = 0, class F>
__device__ __forceinline__ void static_for(F&& f)
{
    if constexpr (I < N) {
        f(ic<I>{});
        static_for<N, I + 1>(f);
    }
}
// after an explicit `s_waitcnt lgkmcnt(0)`: the read's result is defined here (no use moves above it)
__device__ __forceinline__ void tie(u32x4& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void tie(u32x2& v) { asm volatile("" : "+v"(v)); }
__device__ __forceinline__ void tie(uint32_t& v) { asm volatile("" : "+v"(v)); }

}  // namespace phx
