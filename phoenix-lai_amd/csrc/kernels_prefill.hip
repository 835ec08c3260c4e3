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
// tile of up to 128 assignments (four 32-token column tiles; the empty ones are skipped).  Per block,
// the tile's activations (the fp16 copy of their Q8_0 integers that the quantizer writes) are staged
// in LDS once for the four waves (token rows of 40 halves, an 80-byte stride that keeps the 16-byte
// reads free of bank conflicts), with each token's scale as a ready operand entry; the weights and the
// activations stream one block ahead.
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
};

constexpr int MMA_NT = 4;                 // 32-token column tiles per workgroup
constexpr int MMA_TOK = 32 * MMA_NT;      // tile capacity (kMmaTile)
constexpr int MMA_LDS_TOK = 40;           // halves per staged token row
static_assert(MMA_TOK == kMmaTile, "tile capacity");

// eight values of two dwords as an mh8 operand
__device__ __forceinline__ mh8 bias8(uint32_t w0, uint32_t w1, float bias)
{
    const uint4 u = make_uint4(bias_pair(w0, 0, bias), bias_pair(w0, 1, bias), bias_pair(w1, 0, bias),
                               bias_pair(w1, 1, bias));
    return __builtin_bit_cast(mh8, u);
}

// One workgroup's tile: NJ active 32-token column tiles (1..4), every block's MFMAs issued before the
// chain's VALU work.  sx / sdx: the workgroup's LDS staging buffers.
template <int TYPE, int NJ>
__device__ __forceinline__ void mma_tile(const MmaArgs& g, const Tile& tl, int cnt, uint32_t* sx, uint4* sdx,
                                         const uint4& szero)
{
    constexpr int PAY = TYPE == PHX_Q4_0_DEV ? 16 : 32;
    constexpr int XW = MMA_TOK * MMA_LDS_TOK / 2;  // dwords per staging buffer
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r32 = lane & 31, h = lane >> 5;
    const int gI = blockIdx.x * 2 + (wave >> 1), half = wave & 1;
    const bool live = gI < g.rg;  // a wave past the last row group computes a clamped one, stores nothing
    const int nb = g.nb;

    // staging: thread tid brings token tid / 2, halves 16 (tid % 2) .. + 15 of each block of the
    // activations' fp16 copy, and the block's scale as a ready scale-product operand entry
    const int st_tok = tid >> 1, st_part = tid & 1;
    const bool st_valid = st_tok < cnt;
    const int64_t st_row = st_valid ? (int64_t)(g.perm[tl.start + st_tok] / g.act_div) : 0;
    const uint16_t* st_q = g.act.qh + st_row * g.act.qhstride + 16 * st_part;
    const float* st_d = g.act.d + st_row * g.act.dstride;
    uint4 xq0, xq1;
    float xd;
    auto load_x = [&](int b) {
        xq0 = *(const uint4*)(st_q + (int64_t)b * 32);
        xq1 = *(const uint4*)(st_q + (int64_t)b * 32 + 8);
        xd = st_d[b];
    };
    const uint32_t st_mask = st_valid ? ~0u : 0u;  // invalid tokens: zeros
    // unconditional in every thread (both threads of a token write the same scale entry), so the
    // compiler keeps the loads where they are issued instead of sinking them to a conditional use
    auto store_x = [&](int buf) {
        uint32_t* dst = sx + buf * XW + st_tok * (MMA_LDS_TOK / 2) + 8 * st_part;
        *(uint4*)dst = make_uint4(xq0.x & st_mask, xq0.y & st_mask, xq0.z & st_mask, xq0.w & st_mask);
        *(uint4*)(dst + 4) = make_uint4(xq1.x & st_mask, xq1.y & st_mask, xq1.z & st_mask, xq1.w & st_mask);
        sdx[buf * MMA_TOK + st_tok] = make_uint4(f2h_bits(xd) & st_mask, 0u, 0u, 0u);  // xd is an fp16 value
    };

    // weights: lane (row 32 half + r32, h) reads the payload bytes of its k values and its row's fp16
    // scale from the row group's scale groups
    const int gIc = min(gI, g.rg - 1);
    const uint8_t* rgp = g.payload + tl.e * g.mat_pay + gIc * g.rg_pay;
    const int wrow = half * 32 + r32;
    struct WB {
        uint2 q0, q1;  // Q4_0: q0 = bytes 8h..8h+7; Q8_0: q0 = bytes 8h.., q1 = bytes 16 + 8h..
        uint32_t sc;   // fp16 scale bits of the block (row wrow)
    };
    auto load_w = [&](int b, WB& w) {
        const uint8_t* pb = rgp + ((int64_t)b * 64 + wrow) * PAY + 8 * h;
        w.q0 = *(const uint2*)pb;
        w.q1 = TYPE == PHX_Q4_0_DEV ? w.q0 : *(const uint2*)(pb + 16);
        w.sc = *(const uint16_t*)(rgp + g.sc_off + ((int64_t)(b >> 3) * 64 + wrow) * 16 + (b & 7) * 2);
    };

    mf16 S[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
        for (int q = 0; q < 16; q++) S[j][q] = 0.0f;
    const mf16 zero = {};
    const uint32_t hmask = h == 0 ? 0xFFFFu : 0u;  // the scale MFMA's single k sits in lanes 0-31, element 0

    // one block: block b + 1's loads first, then block b from the weights in w and the staged rows;
    // tile j + 1's products go out before tile j's chain, so the matrix cores overlap the VALU work
    WB w, wn;
    load_x(0);
    load_w(0, w);
    store_x(0);
    __syncthreads();
    for (int b = 0; b < nb; b++) {
        const int buf = b & 1;
        load_x(min(b + 1, nb - 1));
        load_w(min(b + 1, nb - 1), wn);
        mh8 A0, A1;
        if (TYPE == PHX_Q4_0_DEV) {
            A0 = bias8(w.q0.x & 0x0F0F0F0Fu, w.q0.y & 0x0F0F0F0Fu, 1032.0f);
            A1 = bias8((w.q0.x >> 4) & 0x0F0F0F0Fu, (w.q0.y >> 4) & 0x0F0F0F0Fu, 1032.0f);
        } else {
            A0 = bias8(w.q0.x ^ 0x80808080u, w.q0.y ^ 0x80808080u, 1152.0f);
            A1 = bias8(w.q1.x ^ 0x80808080u, w.q1.y ^ 0x80808080u, 1152.0f);
        }
        const mh8 Ad = __builtin_bit_cast(mh8, make_uint4(w.sc & hmask, 0u, 0u, 0u));
        const uint32_t* xb = sx + buf * XW;
        auto products = [&](int j, mf16& C, mf16& D) {
            const uint32_t* row = xb + (32 * j + r32) * (MMA_LDS_TOK / 2);
            const mh8 B0 = __builtin_bit_cast(mh8, *(const uint4*)(row + 4 * h));
            const mh8 B1 = __builtin_bit_cast(mh8, *(const uint4*)(row + 8 + 4 * h));
            const mh8 Bd = __builtin_bit_cast(mh8, *(h == 0 ? &sdx[buf * MMA_TOK + 32 * j + r32] : &szero));
            C = __builtin_amdgcn_mfma_f32_32x32x16_f16(A0, B0, zero, 0, 0, 0);
            C = __builtin_amdgcn_mfma_f32_32x32x16_f16(A1, B1, C, 0, 0, 0);
            D = __builtin_amdgcn_mfma_f32_32x32x16_f16(Ad, Bd, zero, 0, 0, 0);
        };
        mf16 C[2], D[2];  // slots j % 2: compile-time after unrolling, so no copies
        products(0, C[0], D[0]);
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            if (j + 1 < NJ) products(j + 1, C[(j + 1) & 1], D[(j + 1) & 1]);
            // the reference chain: sum += (float)isum * (d_w * d_x), in block order
#pragma unroll
            for (int q = 0; q < 16; q++) S[j][q] = S[j][q] + C[j & 1][q] * D[j & 1][q];
        }
        store_x(buf ^ 1);  // that buffer was last read before the previous barrier (after the last block:
                           // a harmless write of a buffer nobody reads again)
        w = wn;
        __syncthreads();
    }

    // results: lane holds rows i_q = 8 (q / 4) + 4 h + (q % 4) of the wave's 32, token column r32
    if (!live) return;
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int sidx = 32 * j + r32;
        if (sidx >= cnt) continue;
        const int64_t a = g.perm[tl.start + sidx];
#pragma unroll
        for (int q = 0; q < 16; q++) {
            const int lg = half * 32 + 8 * (q >> 2) + 4 * h + (q & 3);  // lane within the row group
            if (g.paired) {
                const int col = gI * 32 + (lg & 31);
                if (col < g.split) (lg < 32 ? g.out0 : g.out1)[a * g.out_stride + col] = S[j][q];
            } else {
                const int row = gI * 64 + lg;
                if (row < g.rows) {
                    if (row < g.split) g.out0[a * g.out_stride + row] = S[j][q];
                    else g.out1[a * g.out_stride + row - g.split] = S[j][q];
                }
            }
        }
    }
}

template <int TYPE>
__global__ __launch_bounds__(256) void k_grouped_mfma(MmaArgs g)
{
    __shared__ __align__(16) uint32_t sx[2 * MMA_TOK * MMA_LDS_TOK / 2];  // fp16 token rows of one block
    __shared__ __align__(16) uint4 sdx[2 * MMA_TOK];  // their scales: (fp16 bits, 0, 0, 0) operand entries
    __shared__ __align__(16) uint4 szero;             // the upper lanes' scale operand
    const int tile = blockIdx.y;
    if (tile >= *g.ntiles) return;  // uniform over the workgroup
    if (threadIdx.x == 0) szero = make_uint4(0u, 0u, 0u, 0u);  // visible after mma_tile's first barrier
    const Tile tl = g.tiles[tile];
    const int cnt = min(tl.cnt, MMA_TOK);
    switch ((cnt + 31) / 32) {  // active 32-token column tiles
    case 1: mma_tile<TYPE, 1>(g, tl, cnt, sx, sdx, szero); break;
    case 2: mma_tile<TYPE, 2>(g, tl, cnt, sx, sdx, szero); break;
    case 3: mma_tile<TYPE, 3>(g, tl, cnt, sx, sdx, szero); break;
    default: mma_tile<TYPE, 4>(g, tl, cnt, sx, sdx, szero); break;
    }
}

void launch_grouped_mfma(hipStream_t st, const QMat& w, Act act, const Tile* tiles, const int* ntiles, int max_tiles,
                         const int* perm, int act_div, float* out0, float* out1, int split, int out_stride)
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
    const dim3 grid((w.rg + 1) / 2, max_tiles);
    if (w.type == PHX_Q4_0_DEV) launch(k_grouped_mfma<PHX_Q4_0_DEV>, grid, dim3(256), 0, st, g);
    else launch(k_grouped_mfma<PHX_Q8_0_DEV>, grid, dim3(256), 0, st, g);
}

}  // namespace phx
