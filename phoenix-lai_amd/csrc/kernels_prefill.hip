// Prefill-shaped grouped products on the matrix cores (gfx950 MFMA), Q4_0 and Q8_0 weights.
//
// The reference row dot is, per 32-element block b, sum += (float)isum_b * (d_w * d_x) in block
// order (src/CpuRefGemma.cs:27-36, src/CpuRef.cs:106-115).  Per block and 32 x 32 (row, token) tile:
//   - two v_mfma_f32_32x32x16_f16 give isum_b exactly as floats: the weights enter as the integers
//     q_w - 8 (Q4_0) or q_w (Q8_0) and the activations as their Q8_0 integers, all exact in fp16, and
//     every partial sum is an integer below 2^24, so the fp32 accumulation is exact in any order;
//   - one more v_mfma_f32_32x32x16_f16 with a single nonzero k forms d_w * d_x for the whole tile:
//     both scales are fp16 values, so the products are exact in fp32;
//   - the float chain runs on VALU, one multiply and one add per (row, token, block), in block order,
//     so results equal the CPU reference bit for bit.
//
// Operand layout of v_mfma_f32_32x32x16_f16 (verified on gfx950): A lane l holds row l % 32 and the
// eight k values 8 (l / 32) + e, e = 0..7; B lane l holds column l % 32 and the same k; the 32 x 32
// result C[i][j] sits in lane j + 32 * ((i / 4) % 2), register (i % 4) + 4 * (i / 8).
//
// Work layout: a workgroup of four waves covers two row groups (128 rows; wave w: 32 rows) and one
// tile of up to 128 assignments (four 32-token column tiles; the empty ones are skipped).  Every
// block's operands reach LDS by direct global -> LDS loads (no registers, no staging code) into a ring
// of MMA_RING slots, MMA_RING - 1 blocks ahead of the block being multiplied: the tile's activation
// rows (the fp16 copy of their Q8_0 integers that the quantizer writes) and their scales, the 128
// weight rows' payload and their fp16 scales.  Each wave issues the same five loads per block, so
// its own count of outstanding loads tells when a block has landed; one barrier per block then
// publishes it.  The operands are read from LDS with explicit ds_read instructions whose completion
// the code waits for itself (the compiler would otherwise wait for every outstanding direct load
// before any LDS read).  Activation rows sit in 16-token groups of 1 KB with the four 16-byte parts
// of token t at slot 4 (t % 16) + (part ^ ((t % 16) / 4)), so the 32 lanes of an operand read hit
// 32 distinct bank groups.  A wave keeps one block-sum / scale-product pair (each column's chain
// follows its own products), which holds it to 163 VGPRs: three workgroups per CU (three waves per
// SIMD, 3 x 44 KB of LDS for Q4_0) fill each other's waits.
#include "device_common.h"

namespace phx {

typedef _Float16 mh8 __attribute__((ext_vector_type(8)));
typedef float mf16 __attribute__((ext_vector_type(16)));

struct MmaArgs {
    const uint8_t* payload;
    const uint8_t* scale;
    int64_t mat_pay, mat_sc, rg_pay, sc_off;
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
    // npos > 0: the activations are in expert-list order, block-major: the fp16 integers of (block b,
    // list position p) at act.qh + (b * npos + p) * 32 and its scale at act.d[b * npos + p] (token t
    // of a tile is position tiles.start + t; no perm indirection on the input side)
    int64_t npos;
    // paired gate|up only, when qout.qh is set: e = gelu(g) * u quantized to Q8_0 into qout (the down
    // product's input, one 32-column block per row group) in that list-order layout over qnpos
    // positions, in place of a separate requant pass; only the fp16 integers and the scales are
    // written (what the matrix-core down product reads)
    Act qout;
    int64_t qnpos;
    const float* gelu_tab;
};

constexpr int MMA_NT = 4;                 // 32-token column tiles per workgroup
constexpr int MMA_TOK = 32 * MMA_NT;      // tile capacity (kMmaTile)
static_assert(MMA_TOK == kMmaTile, "tile capacity");

// eight values of two dwords as an mh8 operand
__device__ __forceinline__ mh8 bias8(uint32_t w0, uint32_t w1, float bias)
{
    const uint4 u = make_uint4(bias_pair(w0, 0, bias), bias_pair(w0, 1, bias), bias_pair(w1, 0, bias),
                               bias_pair(w1, 1, bias));
    return __builtin_bit_cast(mh8, u);
}

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void* lds_void_t;
typedef __attribute__((address_space(1))) void* glb_void_t;

constexpr int MMA_RING = 4;  // LDS ring slots: blocks in flight ahead of the one being multiplied
constexpr int MMA_DMA = 5;   // direct loads per wave per block

// LDS ring slot layout (bytes).  A direct load of 1, 2 or 4 bytes writes lane l's value at 4 l from
// the wave's LDS base (16 l for 16-byte loads).
template <int TYPE>
struct MmaSlot {
    static constexpr int PAY = TYPE == PHX_Q4_0_DEV ? 16 : 32;
    static constexpr int ACT = 0;                    // 128 tokens x 64 B, swizzled 16-token groups
    static constexpr int ADX = ACT + MMA_TOK * 64;   // 128 token scales (float)
    static constexpr int WQ = ADX + MMA_TOK * 4;     // 128 weight rows x PAY
    static constexpr int WD = WQ + 128 * PAY;        // 128 weight scales (fp16 in the low half of a dword)
    static constexpr int BYTES = WD + 128 * 4;
};

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
__device__ __forceinline__ uint32_t ds_ru16(uint32_t a)
{
    uint32_t v;
    asm volatile("ds_read_u16 %0, %1" : "=v"(v) : "v"(a));
    return v;
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

// byte offset of (token t, 16-byte part q) in a slot's activation rows
__device__ __forceinline__ uint32_t act_off(int t, int q)
{
    const int tl = t & 15;
    return (uint32_t)((t >> 4) * 1024 + (tl * 4 + (q ^ (tl >> 2))) * 16);
}

// One workgroup's tile: NJ active 32-token column tiles (1..4).  ring: the workgroup's LDS ring.
template <int TYPE, int NJ>
__device__ __forceinline__ void mma_tile(const MmaArgs& g, const Tile& tl, int cnt, unsigned char* ring)
{
    using SL = MmaSlot<TYPE>;
    constexpr int PAY = SL::PAY;
    const int tid = threadIdx.x, lane = tid & 63, r32 = lane & 31, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gI = blockIdx.x * 2 + (wave >> 1), half = wave & 1;
    const bool live = gI < g.rg;  // a wave past the last row group computes a clamped one, stores nothing
    const int nb = g.nb;
    const uint32_t ring0 = (uint32_t)(uintptr_t)(lds_void_t)ring;

    // this wave's five direct loads per block: lane addresses at block 0 and their per-block steps
    // (1) (2) activation rows of tokens 32 w + 16 i + lane / 4, part (lane % 4) ^ (lane / 16)
    const uint16_t* xs[2];
    const bool lst = g.npos > 0;
    const int64_t xstep = lst ? g.npos * 32 : 32, dstep = lst ? g.npos : 1;  // per block
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int t = min(32 * wave + 16 * i + (lane >> 2), cnt - 1);  // past cnt: a valid row, never stored
        const int q = (lane & 3) ^ ((lane >> 4) & 3);
        xs[i] = lst ? g.act.qh + (int64_t)(tl.start + t) * 32 + 8 * q
                    : g.act.qh + (int64_t)(g.perm[tl.start + t] / g.act_div) * g.act.qhstride + 8 * q;
    }
    // (3) token scales of tokens 32 w + lane (lanes 0-31)
    const int td = min(32 * wave + r32, cnt - 1);
    const float* ds = lst ? g.act.d + tl.start + td : g.act.d + (int64_t)(g.perm[tl.start + td] / g.act_div) * g.act.dstride;
    // (4) weight payload: Q4_0 rows 32 half + lane (lanes 0-31), Q8_0 row 32 half + lane / 2, half lane % 2
    const int gIc = min(gI, g.rg - 1);
    const uint8_t* rgp = g.payload + tl.e * g.mat_pay + gIc * g.rg_pay;
    const uint8_t* wq = PAY == 16 ? rgp + (32 * half + r32) * 16 : rgp + (32 * half + (lane >> 1)) * 32 + 16 * (lane & 1);
    // (5) weight scales of rows 32 half + lane (lanes 0-31): fp16 at (b / 8, row) * 16 + (b % 8) * 2
    const uint8_t* wd = rgp + g.sc_off + (32 * half + r32) * 16;

    auto issue = [&](int b) {  // block b (clamped: past the end a harmless reload) into its ring slot
        const int bc = min(b, nb - 1);
        unsigned char* slot = ring + (b % MMA_RING) * SL::BYTES;
        __builtin_amdgcn_global_load_lds((glb_void_t)(xs[0] + bc * xstep),
                                         (lds_void_t)(slot + SL::ACT + (2 * wave) * 1024), 16, 0, 0);
        __builtin_amdgcn_global_load_lds((glb_void_t)(xs[1] + bc * xstep),
                                         (lds_void_t)(slot + SL::ACT + (2 * wave + 1) * 1024), 16, 0, 0);
        if (h == 0) {
            __builtin_amdgcn_global_load_lds((glb_void_t)(ds + bc * dstep), (lds_void_t)(slot + SL::ADX + 128 * wave), 4,
                                             0, 0);
            __builtin_amdgcn_global_load_lds((glb_void_t)(wd + (int64_t)(bc >> 3) * 1024 + (bc & 7) * 2),
                                             (lds_void_t)(slot + SL::WD + 128 * wave), 2, 0, 0);
        }
        if (PAY == 32 || h == 0)
            __builtin_amdgcn_global_load_lds((glb_void_t)(wq + (int64_t)bc * 64 * PAY),
                                             (lds_void_t)(slot + SL::WQ + 32 * PAY * wave), 16, 0, 0);
    };

    mf16 S[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
        for (int q = 0; q < 16; q++) S[j][q] = 0.0f;
    const mf16 zero = {};
    const uint32_t hmask = h == 0 ? 0xFFFFu : 0u;  // the scale MFMA's single k sits in lanes 0-31, element 0

    // the lane's LDS read offsets within a slot
    const uint32_t o_b0 = SL::ACT + act_off(r32, h), o_b1 = SL::ACT + act_off(r32, 2 + h);
    const uint32_t o_dx = SL::ADX + 4 * r32;
    const uint32_t o_wq = SL::WQ + 32 * PAY * wave + PAY * r32 + 8 * h;
    const uint32_t o_wd = SL::WD + 128 * wave + 4 * r32;

    // block b has landed once at most the two later blocks' loads are outstanding; the barrier then
    // publishes it to every wave, and ends every wave's reads of the slot that issue(b + RING - 1)
    // refills (the slot of block b - 1)
    auto land = [&](int b) {
        __builtin_amdgcn_s_waitcnt((MMA_DMA * (MMA_RING - 2)) | (0x7 << 4) | (0xF << 8));
        __builtin_amdgcn_s_barrier();
        issue(b + MMA_RING - 1);
    };
    u32x2 wq0, wq1;
    uint32_t wdv;
    u32x4 B0[2], B1[2];
    uint32_t dx[2];
    uint32_t a_b0, a_b1, a_dx;  // this block's read addresses (tile offsets go in the immediates)
    // the block's first reads: weights, weight scale and tile 0's operands
    auto start_reads = [&](int b) {
        const uint32_t sb = ring0 + (b % MMA_RING) * SL::BYTES;
        a_b0 = sb + o_b0;
        a_b1 = sb + o_b1;
        a_dx = sb + o_dx;
        wq0 = ds_r64(sb + o_wq);
        if (PAY == 32) wq1 = ds_r64<16>(sb + o_wq);
        wdv = ds_ru16(sb + o_wd);
        B0[0] = ds_r128(a_b0);
        B1[0] = ds_r128(a_b1);
        dx[0] = ds_r32(a_dx);
    };
    auto start_wait = [&]() {
        if (PAY == 32) lds_wait(B0[0], B1[0], dx[0], wq0, wq1, wdv);
        else lds_wait(B0[0], B1[0], dx[0], wq0, wdv);
    };
    auto reads = [&](int j) {  // tile j's operands (j: compile-time)
        const int s = j & 1;
        switch (j) {
        case 1: B0[s] = ds_r128<2048>(a_b0); B1[s] = ds_r128<2048>(a_b1); dx[s] = ds_r32<128>(a_dx); break;
        case 2: B0[s] = ds_r128<4096>(a_b0); B1[s] = ds_r128<4096>(a_b1); dx[s] = ds_r32<256>(a_dx); break;
        default: B0[s] = ds_r128<6144>(a_b0); B1[s] = ds_r128<6144>(a_b1); dx[s] = ds_r32<384>(a_dx); break;
        }
    };
    u32x4 bd = {0u, 0u, 0u, 0u}, ad = {0u, 0u, 0u, 0u};  // scale operands: one nonzero element

#pragma unroll
    for (int b = 0; b < MMA_RING - 1; b++) issue(b);
    land(0);
    start_reads(0);
    start_wait();
    for (int b = 0; b < nb; b++) {
        mh8 A0, A1;
        if (TYPE == PHX_Q4_0_DEV) {
            A0 = bias8(wq0.x & 0x0F0F0F0Fu, wq0.y & 0x0F0F0F0Fu, 1032.0f);
            A1 = bias8((wq0.x >> 4) & 0x0F0F0F0Fu, (wq0.y >> 4) & 0x0F0F0F0Fu, 1032.0f);
        } else {
            A0 = bias8(wq0.x ^ 0x80808080u, wq0.y ^ 0x80808080u, 1152.0f);
            A1 = bias8(wq1.x ^ 0x80808080u, wq1.y ^ 0x80808080u, 1152.0f);
        }
        ad.x = wdv & hmask;
        const mh8 Ad = __builtin_bit_cast(mh8, ad);
        mf16 C, D;  // one slot: each column's chain follows its own products (three waves per SIMD
                    // fill the wait; a second slot would cost the third wave's registers)
        auto products = [&](int j) {
            const int s = j & 1;
            // the token scale is an fp16 value: the conversion is exact
            bd.x = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)__uint_as_float(dx[s])) & hmask;
            C = __builtin_amdgcn_mfma_f32_32x32x16_f16(A0, __builtin_bit_cast(mh8, B0[s]), zero, 0, 0, 0);
            C = __builtin_amdgcn_mfma_f32_32x32x16_f16(A1, __builtin_bit_cast(mh8, B1[s]), C, 0, 0, 0);
            D = __builtin_amdgcn_mfma_f32_32x32x16_f16(Ad, __builtin_bit_cast(mh8, bd), zero, 0, 0, 0);
        };
        if (NJ > 1) reads(1);
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            if (j > 0) {
                const int s = j & 1;
                lds_wait(B0[s], B1[s], dx[s]);
            }
            products(j);
            if (j + 2 < NJ) reads(j + 2);
            if (j == NJ - 1) {
                // the next block lands and its first reads go out behind this block's last chain (after
                // the last block: a harmless extra barrier and reads of a slot nobody uses)
                land(b + 1);
                start_reads(b + 1);
            }
            // keep the program order: the reads ahead of the chain, the chain before the next column
            __builtin_amdgcn_sched_barrier(0);
            // the reference chain: sum += (float)isum * (d_w * d_x), in block order
#pragma unroll
            for (int q = 0; q < 16; q++) S[j][q] = S[j][q] + C[q] * D[q];
            asm volatile("" : "+v"(S[j]));  // the chain stays here, not sunk towards its next use
            __builtin_amdgcn_sched_barrier(0);
            if (j == NJ - 1) start_wait();  // in the reads' basic block: the loop carries landed values
        }
    }
    // the loads issued past the last block land in this workgroup's LDS: let them finish before it ends
    __builtin_amdgcn_s_waitcnt(0);

    if (g.qout.qh) {  // uniform: the requant epilogue (src/GemmaCpu.cs:415, src/CpuRef.cs:49-62)
        // the gate wave of each pair (half 0) forms gelu(g) (src/CpuRefGemma.cs:85-92: the table lookups
        // of all its values issued together) and hands it to the up wave through the ring
        __syncthreads();  // every wave is done with the ring
        float* xg = (float*)ring + (wave >> 1) * (MMA_NT * 16 * 64);
        if (half == 0) {
            float tv[NJ][16];
#pragma unroll
            for (int j = 0; j < NJ; j++)
#pragma unroll
                for (int q = 0; q < 16; q++) tv[j][q] = g.gelu_tab[f2h_bits(S[j][q])];
#pragma unroll
            for (int j = 0; j < NJ; j++)
#pragma unroll
                for (int q = 0; q < 16; q++) {
                    const float v = S[j][q];
                    xg[(j * 16 + q) * 64 + lane] = v <= -10.0f ? 0.0f : (v >= 10.0f ? v : tv[j][q]);
                }
        }
        __syncthreads();
        if (half == 1 && live) {
            const Act& o = g.qout;
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                // lane (r32, h): token column r32 of tile j, block columns 8 (q / 4) + 4 h + q % 4
                float e[16], am = 0.0f;
#pragma unroll
                for (int q = 0; q < 16; q++) {
                    const int col = gI * 32 + 8 * (q >> 2) + 4 * h + (q & 3);
                    e[q] = col < g.split ? xg[(j * 16 + q) * 64 + lane] * S[j][q] : 0.0f;
                    am = fmaxf(am, fabsf(e[q]));
                }
                am = fmaxf(am, __shfl_xor(am, 32, 64));  // the other 16 columns: lane r32 + 32 (1 - 2 h)
                const float dd = am / 127.0f;
                const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
                // the integers as exact fp16 (signed bytes through the 1152 bias), four per column group
                uint32_t w[4][2];
#pragma unroll
                for (int g4 = 0; g4 < 4; g4++) {
                    const int q0 = (int)roundf(e[4 * g4] * id), q1 = (int)roundf(e[4 * g4 + 1] * id),
                              q2 = (int)roundf(e[4 * g4 + 2] * id), q3 = (int)roundf(e[4 * g4 + 3] * id);
                    const uint32_t u = (uint32_t)((q0 & 0xFF) | ((q1 & 0xFF) << 8) | ((q2 & 0xFF) << 16) |
                                                  ((unsigned)q3 << 24)) ^ 0x80808080u;
                    w[g4][0] = bias_pair(u, 0, 1152.0f);
                    w[g4][1] = bias_pair(u, 1, 1152.0f);
                }
                // this lane writes columns 16 h .. 16 h + 15: groups 2 h and 2 h + 1 of both halves (the
                // partner lane's half from it)
                const uint32_t s0 = h ? w[0][0] : w[2][0], s1 = h ? w[0][1] : w[2][1];
                const uint32_t s2 = h ? w[1][0] : w[3][0], s3 = h ? w[1][1] : w[3][1];
                const uint32_t p0 = (uint32_t)__shfl_xor((int)s0, 32, 64), p1 = (uint32_t)__shfl_xor((int)s1, 32, 64);
                const uint32_t p2 = (uint32_t)__shfl_xor((int)s2, 32, 64), p3 = (uint32_t)__shfl_xor((int)s3, 32, 64);
                const uint4 lo = h ? make_uint4(p0, p1, w[2][0], w[2][1]) : make_uint4(w[0][0], w[0][1], p0, p1);
                const uint4 hi = h ? make_uint4(p2, p3, w[3][0], w[3][1]) : make_uint4(w[1][0], w[1][1], p2, p3);
                const int sidx = 32 * j + r32;
                if (sidx < cnt) {
                    const int64_t pos = (int64_t)gI * g.qnpos + tl.start + sidx;
                    uint16_t* hq = o.qh + pos * 32 + 16 * h;
                    *(uint4*)hq = lo;
                    *(uint4*)(hq + 8) = hi;
                    if (h == 0) o.d[pos] = h2f(f2h_bits(dd));
                }
            }
        }
    }

    // results: lane holds rows i_q = 8 (q / 4) + 4 h + (q % 4) of the wave's 32, token column r32
    if (!live) return;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int sidx = 32 * j + r32;
        if (sidx >= cnt) continue;
        const int64_t a = g.perm[tl.start + sidx];
        // four consecutive rows (columns of the output row a) per q4: one 16-byte store where the four
        // lie inside the output and the row stride keeps them aligned, else element by element
        const bool vec = (g.out_stride & 3) == 0;
#pragma unroll
        for (int q4 = 0; q4 < 4; q4++) {
            const int lg0 = half * 32 + 8 * q4 + 4 * h;  // lane within the row group of the first of four
            const float4 v = make_float4(S[j][4 * q4], S[j][4 * q4 + 1], S[j][4 * q4 + 2], S[j][4 * q4 + 3]);
            if (g.paired) {
                const int col = gI * 32 + (lg0 & 31);
                float* dst = (half ? g.out1 : g.out0) + a * g.out_stride + col;
                if (vec && col + 3 < g.split) *(float4*)dst = v;
                else
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        if (col + i < g.split) dst[i] = S[j][4 * q4 + i];
            } else {
                const int row = gI * 64 + lg0;
                if (vec && row + 3 < min(g.rows, g.split)) *(float4*)(g.out0 + a * g.out_stride + row) = v;
                else
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int r = row + i;
                        if (r < g.rows) {
                            if (r < g.split) g.out0[a * g.out_stride + r] = S[j][4 * q4 + i];
                            else g.out1[a * g.out_stride + r - g.split] = S[j][4 * q4 + i];
                        }
                    }
            }
        }
    }
}

template <int TYPE>
__global__ __launch_bounds__(256, 3) void k_grouped_mfma(MmaArgs g)
{
    __shared__ __align__(16) unsigned char ring[MMA_RING * MmaSlot<TYPE>::BYTES];
    const int tile = blockIdx.y;
    if (tile >= *g.ntiles) return;  // uniform over the workgroup
    const Tile tl = g.tiles[tile];
    const int cnt = min(tl.cnt, MMA_TOK);
    switch ((cnt + 31) / 32) {  // active 32-token column tiles
    case 1: mma_tile<TYPE, 1>(g, tl, cnt, ring); break;
    case 2: mma_tile<TYPE, 2>(g, tl, cnt, ring); break;
    case 3: mma_tile<TYPE, 3>(g, tl, cnt, ring); break;
    default: mma_tile<TYPE, 4>(g, tl, cnt, ring); break;
    }
}

void launch_grouped_mfma(hipStream_t st, const QMat& w, Act act, const Tile* tiles, const int* ntiles, int max_tiles,
                         const int* perm, int act_div, float* out0, float* out1, int split, int out_stride,
                         int64_t npos, const Act* qout, int64_t qnpos, const float* gelu_tab)
{
    MmaArgs g;
    g.payload = w.payload;
    g.scale = w.scale;
    g.mat_pay = w.mat_pay_stride();
    g.rg_pay = w.rg_pay;
    g.sc_off = w.sc8_off();
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
    g.npos = npos;
    g.qout = qout && w.paired ? *qout : Act{};
    g.qnpos = qnpos;
    g.gelu_tab = gelu_tab;
    const dim3 grid((w.rg + 1) / 2, max_tiles);
    if (w.type == PHX_Q4_0_DEV) launch(k_grouped_mfma<PHX_Q4_0_DEV>, grid, dim3(256), 0, st, g);
    else launch(k_grouped_mfma<PHX_Q8_0_DEV>, grid, dim3(256), 0, st, g);
}

}  // namespace phx
