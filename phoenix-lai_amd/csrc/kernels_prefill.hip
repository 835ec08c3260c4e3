// Prefill-shaped grouped products on the matrix cores (gfx950 MFMA), Q4_0 and Q8_0 weights.
//
// The reference row dot is, per 32-element block b, sum += (float)isum_b * (d_w * d_x) in block
// order (src/CpuRefGemma.cs:27-36, src/CpuRef.cs:106-115).  Here the integer block sums of a
// 32-row x 32-token tile come from one v_mfma_i32_32x32x32_i8 per block (exact int32), and the
// float chain runs on VALU in block order for every (row, token), so results equal the CPU
// reference bit for bit.  Q4_0 nibbles enter the MFMA as 0..15; a second MFMA with a constant -8
// operand adds -8 * sum_k q_x, giving the signed block sums without per-element work.
//
// Operand layout (verified on gfx950): A lane l holds row l % 32 and 16 of the block's 32 k values
// (lanes 0-31 one set, 32-63 the other); B lane l holds token l % 32 and the same k set; the
// 32 x 32 result C[i][j] sits in lane j + 32 * ((i / 4) % 2), register (i % 4) + 4 * (i / 8).  Q4_0
// lanes 0-31 take the low nibbles (elements 0-15) and 32-63 the high nibbles (16-31).
#include "device_common.h"

namespace phx {

typedef int mv4i __attribute__((ext_vector_type(4)));
typedef int mv16i __attribute__((ext_vector_type(16)));

struct MmaArgs {
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

constexpr int MMA_NTOK = 2;  // 32-token column tiles per wave: tiles of up to 64 assignments

template <int TYPE>
__global__ __launch_bounds__(256) void k_grouped_mfma(MmaArgs g)
{
    const int tile = blockIdx.y;
    if (tile >= *g.ntiles) return;
    const Tile tl = g.tiles[tile];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int r32 = lane & 31, h = lane >> 5;
    const int R0 = blockIdx.x * 128 + wave * 32;  // first (repacked) row of this wave's slice
    const int gI = R0 >> 6, half = (R0 >> 5) & 1;
    if (gI >= g.rg) return;  // no barriers below: a wave past the last row group just stops
    constexpr int PAY = TYPE == PHX_Q4_0_DEV ? 16 : 32;
    const int nb = g.nb;

    // the tile's tokens: column r32 of each 32-token column tile
    int orow[MMA_NTOK];
    int64_t arow[MMA_NTOK];
    bool valid[MMA_NTOK];
#pragma unroll
    for (int j = 0; j < MMA_NTOK; j++) {
        const int s = 32 * j + r32;
        valid[j] = s < tl.cnt;
        orow[j] = valid[j] ? g.perm[tl.start + s] : 0;
        arow[j] = orow[j] / g.act_div;
    }
    const uint8_t* pay = g.payload + tl.e * g.mat_pay + gI * g.rg_pay + (half * 32 + r32) * PAY;
    const uint16_t* scl = (const uint16_t*)(g.scale + tl.e * g.mat_sc) + (int64_t)gI * nb * 64 + half * 32 + 4 * h;
    const mv4i neg8 = {(int)0xF8F8F8F8u, (int)0xF8F8F8F8u, (int)0xF8F8F8F8u, (int)0xF8F8F8F8u};
    const mv16i zero = {};

    float S[MMA_NTOK][16];
#pragma unroll
    for (int j = 0; j < MMA_NTOK; j++)
#pragma unroll
        for (int q = 0; q < 16; q++) S[j][q] = 0.0f;

    // operands of one block, loaded one block ahead of their use (software pipelining)
    struct Stage {
        uint4 w;               // Q4_0: the row's 16 payload bytes; Q8_0: this lane's 16 of 32
        uint2 sc[4];           // fp16 scales of the 16 result rows
        mv4i B[MMA_NTOK];
        float dx[MMA_NTOK];
    };
    auto load = [&](int b, Stage& st) {
        st.w = *(const uint4*)(pay + (int64_t)b * 64 * PAY + (TYPE == PHX_Q4_0_DEV ? 0 : 16 * h));
#pragma unroll
        for (int qq = 0; qq < 4; qq++) st.sc[qq] = *(const uint2*)(scl + (int64_t)b * 64 + 8 * qq);
#pragma unroll
        for (int j = 0; j < MMA_NTOK; j++) {
            if (valid[j]) {
                st.B[j] = *(const mv4i*)(g.act.q + arow[j] * g.act.qstride + b * 32 + 16 * h);
                st.dx[j] = g.act.d[arow[j] * g.act.dstride + b];
            } else {
                st.B[j] = mv4i{0, 0, 0, 0};
                st.dx[j] = 0.0f;
            }
        }
    };
    auto compute = [&](const Stage& st) {
        mv4i A;
        if (TYPE == PHX_Q4_0_DEV) {
            const unsigned sh = h ? 4u : 0u;
            A.x = (int)((st.w.x >> sh) & 0x0F0F0F0Fu);
            A.y = (int)((st.w.y >> sh) & 0x0F0F0F0Fu);
            A.z = (int)((st.w.z >> sh) & 0x0F0F0F0Fu);
            A.w = (int)((st.w.w >> sh) & 0x0F0F0F0Fu);
        } else {
            A = mv4i{(int)st.w.x, (int)st.w.y, (int)st.w.z, (int)st.w.w};
        }
        float dw[16];
#pragma unroll
        for (int qq = 0; qq < 4; qq++) {
            dw[4 * qq + 0] = h2f(st.sc[qq].x & 0xFFFFu);
            dw[4 * qq + 1] = h2f(st.sc[qq].x >> 16);
            dw[4 * qq + 2] = h2f(st.sc[qq].y & 0xFFFFu);
            dw[4 * qq + 3] = h2f(st.sc[qq].y >> 16);
        }
#pragma unroll
        for (int j = 0; j < MMA_NTOK; j++) {
            mv16i C = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, st.B[j], zero, 0, 0, 0);
            if (TYPE == PHX_Q4_0_DEV) C = __builtin_amdgcn_mfma_i32_32x32x32_i8(neg8, st.B[j], C, 0, 0, 0);
            // the reference chain: sum += (float)isum * (d_w * d_x), in block order
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const float dd = dw[q] * st.dx[j];
                S[j][q] = S[j][q] + (float)C[q] * dd;
            }
        }
    };
    Stage s0, s1;
    load(0, s0);
    int b = 0;
    for (; b + 2 <= nb; b += 2) {
        load(b + 1, s1);
        compute(s0);
        if (b + 2 < nb) load(b + 2, s0);
        compute(s1);
    }
    if (b < nb) compute(s0);  // odd block count: the last block is in s0

    // results: lane holds rows i_q = 8 (q / 4) + 4 h + (q % 4) of the slice, token column r32
#pragma unroll
    for (int j = 0; j < MMA_NTOK; j++) {
        if (!valid[j]) continue;
        const int64_t a = orow[j];
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

void launch_grouped_mfma(hipStream_t st, const QMat& w, Act act, const Tile* tiles, const int* ntiles, int max_tiles,
                         const int* perm, int act_div, float* out0, float* out1, int split, int out_stride)
{
    MmaArgs g;
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
    const dim3 grid((w.rg + 1) / 2, max_tiles);
    if (w.type == PHX_Q4_0_DEV) launch(k_grouped_mfma<PHX_Q4_0_DEV>, grid, dim3(256), 0, st, g);
    else launch(k_grouped_mfma<PHX_Q8_0_DEV>, grid, dim3(256), 0, st, g);
}

}  // namespace phx
