// Prefill-shaped grouped products on the matrix cores (gfx950 MFMA): Q4_0 and Q8_0 weights
// (k_grouped_mfma), Q4_K and Q6_K weights (k_grouped_kmma, further down).
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

constexpr int MMA_RING = 4;  // LDS ring slots: blocks in flight ahead of the one being multiplied

// LDS ring slot layout (bytes).  A direct load of 1, 2 or 4 bytes writes lane l's value at 4 l from
// the wave's LDS base (16 l for 16-byte loads).
// Weight scales: Q4_0 rows take their fp16 scales from the row group's scale groups (16 bytes = 8 blocks
// per row) into a two-slot scale ring beside the block ring, one load per wave every 8 blocks (SG); Q8_0
// rows (whose larger payload leaves no LDS for that ring at three workgroups per CU) one 2-byte load per
// block into the slot (WD).  The direct loads' address processing bounds the kernel, so every load
// instruction saved counts.
template <int TYPE>
struct MmaSlot {
    static constexpr int PAY = TYPE == PHX_Q4_0_DEV ? 16 : 32;
    static constexpr bool SG = TYPE == PHX_Q4_0_DEV;
    static constexpr int DMA = SG ? 4 : 5;           // direct loads per wave per block (scale groups aside)
    static constexpr int ACT = 0;                    // 128 tokens x 64 B, swizzled 16-token groups
    static constexpr int ADX = ACT + MMA_TOK * 64;   // 128 token scales (float)
    static constexpr int WQ = ADX + MMA_TOK * 4;     // 128 weight rows x PAY
    static constexpr int WD = WQ + 128 * PAY;        // (Q8_0) 128 weight scales (fp16 in the low half of a dword)
    static constexpr int BYTES = WD + (SG ? 0 : 128 * 4);
    static constexpr int SR = MMA_RING * BYTES;      // (Q4_0) scale ring: [2 groups][4 waves][32 rows][8 fp16]
    static constexpr int LDS = SR + (SG ? 2 * 4 * 512 : 0);
};

// byte offset of (token t, 16-byte part q) in a slot's activation rows
__device__ __forceinline__ uint32_t act_off(int t, int q)
{
    const int tl = t & 15;
    return (uint32_t)((t >> 4) * 1024 + (tl * 4 + (q ^ (tl >> 2))) * 16);
}

// One workgroup's tile: NJ active 32-token column tiles (1..4).  ring: the workgroup's LDS ring.
template <int TYPE, int NJ>
__device__ __forceinline__ void mma_tile(const MmaArgs& g, const Tile& tl, int cnt, unsigned char* ring, int bx)
{
    using SL = MmaSlot<TYPE>;
    constexpr int PAY = SL::PAY;
    const int tid = threadIdx.x, lane = tid & 63, r32 = lane & 31, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gI = bx * 2 + (wave >> 1), half = wave & 1;
    const bool live = gI < g.rg;  // a wave past the last row group computes a clamped one, stores nothing
    const int nb = g.nb;
    const uint32_t ring0 = (uint32_t)(uintptr_t)(lds_void_t)ring;

    // this wave's five direct loads per block, as buffer -> LDS loads: each lane's byte offset at block 0
    // (a VGPR, the same for every block) and the block's uniform offset (an SGPR)
    const bool lst = g.npos > 0;
    const uint32_t xstep = lst ? (uint32_t)g.npos * 64u : 64u, dstep = lst ? (uint32_t)g.npos * 4u : 4u;  // bytes per block
    // (1) (2) activation rows of tokens 32 w + 16 i + lane / 4, part (lane % 4) ^ (lane / 16)
    uint32_t vx[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int t = min(32 * wave + 16 * i + (lane >> 2), cnt - 1);  // past cnt: a valid row, never stored
        const int q = (lane & 3) ^ ((lane >> 4) & 3);
        const int64_t row = lst ? (int64_t)(tl.start + t) * 32 : (int64_t)(g.perm[tl.start + t] / g.act_div) * g.act.qhstride;
        vx[i] = (uint32_t)(2 * (row + 8 * q));
    }
    // (3) token scales of tokens 32 w + lane (lanes 0-31)
    const int td = min(32 * wave + r32, cnt - 1);
    const uint32_t vds = (uint32_t)(4 * (lst ? (int64_t)tl.start + td : (int64_t)(g.perm[tl.start + td] / g.act_div) * g.act.dstride));
    // (4) weight payload: Q4_0 rows 32 half + lane (lanes 0-31), Q8_0 row 32 half + lane / 2, half lane % 2;
    // (5) weight scales of rows 32 half + lane (lanes 0-31): fp16 at (b / 8, row) * 16 + (b % 8) * 2
    const int gIc = min(gI, g.rg - 1);
    const __amdgpu_buffer_rsrc_t r_act = buf_rsrc(g.act.qh), r_ds = buf_rsrc(g.act.d);
    const __amdgpu_buffer_rsrc_t r_w = buf_rsrc(g.payload + tl.e * g.mat_pay + gIc * g.rg_pay);
    const uint32_t vwq = PAY == 16 ? (32 * half + r32) * 16 : (32 * half + (lane >> 1)) * 32 + 16 * (lane & 1);
    const uint32_t vwd = (uint32_t)g.sc_off + (32 * half + r32) * 16;

    // block b (clamped: past the end a harmless reload) into ring slot S = b % MMA_RING; with SG, at the
    // first block of each group of 8 (before the block's own loads, so it lands first) the group's weight
    // scales into scale slot (b / 8) % 2, whose previous group ended eight blocks earlier
    auto issue = [&](auto SC, int b) {
        constexpr int S = decltype(SC)::value;
        const uint32_t bc = (uint32_t)min(b, nb - 1);
        unsigned char* slot = ring + S * SL::BYTES;
        const uint32_t sx = bc * xstep;
        if constexpr (SL::SG) {
            if ((b & 7) == 0 && h == 0)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(
                    r_w, (lds_void_t)(ring + SL::SR + ((b >> 3) & 1) * 2048 + 512 * wave), 16, vwd,
                    (uint32_t)min(b >> 3, (nb - 1) >> 3) * 1024, 0, 0);
        }
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r_act, (lds_void_t)(slot + SL::ACT + (2 * wave) * 1024), 16, vx[0], sx, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r_act, (lds_void_t)(slot + SL::ACT + (2 * wave + 1) * 1024), 16, vx[1], sx,
                                                 0, 0);
        if (h == 0) {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r_ds, (lds_void_t)(slot + SL::ADX + 128 * wave), 4, vds, bc * dstep, 0, 0);
            if constexpr (!SL::SG)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(r_w, (lds_void_t)(slot + SL::WD + 128 * wave), 2, vwd,
                                                         (bc >> 3) * 1024 + (bc & 7) * 2, 0, 0);
        }
        if (PAY == 32 || h == 0)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r_w, (lds_void_t)(slot + SL::WQ + 32 * PAY * wave), 16, vwq,
                                                     bc * 64 * PAY, 0, 0);
    };

    mf16 S[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++)
#pragma unroll
        for (int q = 0; q < 16; q++) S[j][q] = 0.0f;
    const mf16 zero = {};
    const uint32_t hmask = h == 0 ? 0xFFFFu : 0u;  // the scale MFMA's single k sits in lanes 0-31, element 0

    // the lane's LDS read addresses in slot 0 (slot S: + S * BYTES in the immediate offset)
    static_assert(3 * SL::BYTES + SL::WD + 128 * 4 < 65536, "ring offsets fit the LDS immediate");
    // the weight scale of block b: the ring slot's (Q8_0) or the scale ring's (Q4_0: a VGPR offset per block)
    const uint32_t A_SG = ring0 + SL::SR + 512 * wave + 16 * r32;
    auto wd_read = [&](auto SC, int b) -> uint32_t {
        if constexpr (SL::SG) return ds_ru16<0>(A_SG + (uint32_t)(((b >> 3) & 1) * 2048 + (b & 7) * 2));
        else return ds_ru16<decltype(SC)::value * SL::BYTES>(ring0 + SL::WD + 128 * wave + 4 * r32);
    };
    const uint32_t A_B0 = ring0 + SL::ACT + act_off(r32, h), A_B1 = ring0 + SL::ACT + act_off(r32, 2 + h);
    const uint32_t A_DX = ring0 + SL::ADX + 4 * r32;
    const uint32_t A_WQ = ring0 + SL::WQ + 32 * PAY * wave + PAY * r32 + 8 * h;

    // block b has landed once at most the two later blocks' loads are outstanding; the barrier then
    // publishes it to every wave, and ends every wave's reads of the slot that issue(b + RING - 1)
    // refills (the slot of block b - 1)
    auto land = [&](auto SC, int b) {  // S = b % MMA_RING
        constexpr int S = decltype(SC)::value;
        // at most the two later blocks' loads outstanding (a scale-group load among them only makes the
        // wait a little longer: it is older than its block's loads)
        __builtin_amdgcn_s_waitcnt((SL::DMA * (MMA_RING - 2)) | (0x7 << 4) | (0xF << 8));
        __builtin_amdgcn_s_barrier();
        issue(ic<(S + MMA_RING - 1) % MMA_RING>{}, b + MMA_RING - 1);
    };
    u32x2 wq0, wq1;
    uint32_t wdv;
    u32x4 B0[2], B1[2];
    uint32_t dx[2];
    // block b's first reads: weights, weight scale and tile 0's operands
    auto start_reads = [&](auto SC, int b) {
        constexpr int O = decltype(SC)::value * SL::BYTES;
        wq0 = ds_r64<O>(A_WQ);
        if (PAY == 32) wq1 = ds_r64<O + 16>(A_WQ);
        wdv = wd_read(SC, b);
        B0[0] = ds_r128<O>(A_B0);
        B1[0] = ds_r128<O>(A_B1);
        dx[0] = ds_r32<O>(A_DX);
    };
    auto start_wait = [&]() {
        if (PAY == 32) lds_wait(B0[0], B1[0], dx[0], wq0, wq1, wdv);
        else lds_wait(B0[0], B1[0], dx[0], wq0, wdv);
    };
    auto reads = [&](auto SC, auto JC) {  // tile j's operands in slot S
        constexpr int O = decltype(SC)::value * SL::BYTES, j = decltype(JC)::value, s = j & 1;
        B0[s] = ds_r128<O + 2048 * j>(A_B0);
        B1[s] = ds_r128<O + 2048 * j>(A_B1);
        dx[s] = ds_r32<O + 128 * j>(A_DX);
    };
    u32x4 bd = {0u, 0u, 0u, 0u}, ad = {0u, 0u, 0u, 0u};  // scale operands: one nonzero element

    // block b (in slot S = b % MMA_RING, its first operands already read)
    auto block = [&](auto SC, int b) {
        constexpr int S1 = (decltype(SC)::value + 1) % MMA_RING;  // the next block's slot
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
        if (NJ > 1) reads(SC, ic<1>{});
        static_for<NJ>([&](auto JC) {
            constexpr int j = decltype(JC)::value;
            if (j > 0) {
                constexpr int s = j & 1;
                lds_wait(B0[s], B1[s], dx[s]);
            }
            products(j);
            if constexpr (j + 2 < NJ) reads(SC, ic<j + 2>{});
            if constexpr (j == NJ - 1) {
                // the next block lands and its first reads go out behind this block's last chain (after
                // the last block: a harmless extra barrier and reads of a slot nobody uses)
                land(ic<S1>{}, b + 1);
                start_reads(ic<S1>{}, b + 1);
            }
            // keep the program order: the reads ahead of the chain, the chain before the next column
            __builtin_amdgcn_sched_barrier(0);
            // the reference chain: sum += (float)isum * (d_w * d_x), in block order
#pragma unroll
            for (int q = 0; q < 16; q++) S[j][q] = S[j][q] + C[q] * D[q];
            asm volatile("" : "+v"(S[j]));  // the chain stays here, not sunk towards its next use
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (j == NJ - 1) start_wait();  // in the reads' basic block: the loop carries landed values
        });
    };

    issue(ic<0>{}, 0);
    issue(ic<1>{}, 1);
    issue(ic<2>{}, 2);
    // the ring's slots by unrolling: every LDS offset is an immediate
    static_assert(MMA_RING == 4, "the block loop is unrolled by the ring size");
    land(ic<0>{}, 0);
    start_reads(ic<0>{}, 0);
    start_wait();
    for (int b = 0; b < nb; b += 4) {
        block(ic<0>{}, b);
        if (b + 1 < nb) block(ic<1>{}, b + 1);
        if (b + 2 < nb) block(ic<2>{}, b + 2);
        if (b + 3 < nb) block(ic<3>{}, b + 3);
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

    // results: lane holds rows i_q = 8 (q / 4) + 4 h + (q % 4) of the wave's 32, token column r32 (a
    // paired launch without g and u outputs ends with its requant)
    if (!live || (g.paired && !g.out0)) return;
    // the lane's assignment indices, every load before the first store (a store's wait would otherwise
    // hold the next index's load back)
    int pa[NJ];
#pragma unroll
    for (int j = 0; j < NJ; j++) pa[j] = g.perm[tl.start + min(32 * j + r32, cnt - 1)];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int sidx = 32 * j + r32;
        if (sidx >= cnt) continue;
        const int64_t a = pa[j];
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

// XCD-aware order of the grouped products' grid (gridDim.x row-group pairs by tile slots, the slots
// padded to a multiple of 8): the dispatcher hands workgroup L = y * gridDim.x + x to XCD L % 8, and
// here workgroup L takes tile 8 (k / gridDim.x) + L % 8 and row-group pair k % gridDim.x, k = L / 8 (one
// to one).  A tile's pairs then run on one XCD, one after another, so its activation rows reach that
// XCD's L2 once instead of once in every XCD; the tiles still go out in list order (longest first),
// dealt round robin over the XCDs.
__device__ __forceinline__ int xcd_tile(int* bx)
{
    const int gx = gridDim.x, L = blockIdx.y * gx + blockIdx.x, k = L >> 3;
    *bx = k % gx;
    return 8 * (k / gx) + (L & 7);
}
inline int xcd_tile_slots(int max_tiles) { return (max_tiles + 7) / 8 * 8; }

template <int TYPE>
__global__ __launch_bounds__(256, 3) void k_grouped_mfma(MmaArgs g)
{
    __shared__ __align__(16) unsigned char ring[MmaSlot<TYPE>::LDS];
    int bx;
    const int tile = xcd_tile(&bx);
    if (tile >= *g.ntiles) return;  // uniform over the workgroup
    const Tile tl = g.tiles[tile];
    const int cnt = min(tl.cnt, MMA_TOK);
#ifdef PHX_TIMELINE
    // start and end of each workgroup: entries 2 f, 2 f + 1 of f = tile * gridDim.x + row-group pair (down
    // products: from entry 16384)
    const int wgf = tile * gridDim.x + bx, tbase = g.paired ? 0 : 16384;
    if (threadIdx.x == 0 && wgf < 8192) phx_tl[tbase + 2 * wgf] = wall_clock64();
#endif
    switch ((cnt + 31) / 32) {  // active 32-token column tiles
    case 1: mma_tile<TYPE, 1>(g, tl, cnt, ring, bx); break;
    case 2: mma_tile<TYPE, 2>(g, tl, cnt, ring, bx); break;
    case 3: mma_tile<TYPE, 3>(g, tl, cnt, ring, bx); break;
    default: mma_tile<TYPE, 4>(g, tl, cnt, ring, bx); break;
    }
#ifdef PHX_TIMELINE
    if (threadIdx.x == 0 && wgf < 8192) phx_tl[tbase + 2 * wgf + 1] = wall_clock64();
#endif
}

// ---------------------------------------------------------------------------- tolerance mode
// The products of PHX_FLAG_FAST_MATH, after the reference's own GPU prefill (src/KernelsCoop.cs:1-11:
// weights dequantized to f16, f16 activations, f32 accumulation over the whole row on the matrix
// units): the block scales are folded into the operands, (q_w - 8) * d_w (Q4_0) or q_w * d_w (Q8_0) and
// q_x * d_x, each rounded once to fp16, and every row accumulates in fp32 across all its blocks: two
// v_mfma_f32_32x32x16_f16 per block and (32-row, 32-token) tile, no per-block VALU chain.  Results then
// differ from the CPU reference by the operands' fp16 rounding (about 2^-12 of each term).
//
// Work layout: a workgroup of four waves covers four row groups (256 rows; wave w: row group 4 x + w,
// both of its 32-row halves: gate and up of a paired row group) and one tile of up to 128 assignments,
// so each block of the tile's activations leaves L2 once per 256 rows.  Per block every wave issues the
// same direct loads into a ring slot (its share of the activations and their scales, its row group's
// payload and, for Q8_0, its scales; Q4_0 scales come once per 8 blocks into a two-slot scale ring),
// MMA_RING - 1 blocks ahead; after one barrier per block a wave reads its two weight tiles and the
// tile's activation operands, folds the scales (fp16 products) and issues 4 NJ MFMAs, each column
// tile's two k-halves 2 NJ MFMAs apart.  Two workgroups per CU (two waves per SIMD: 128 accumulator
// registers per wave) take turns between the matrix cores and the reads and folds.  A paired launch's
// wave holds gate and up of the same 32 columns, so the GELU-gated Q8_0 requant of the down input runs
// in its registers.
template <int TYPE>
struct CoopSlot {
    static constexpr int PAY = TYPE == PHX_Q4_0_DEV ? 16 : 32;
    static constexpr bool SG = TYPE == PHX_Q4_0_DEV;
    static constexpr int WL = PAY / 16;                // payload loads per wave and block (1 KB each)
    static constexpr int DMA = 2 + WL + (SG ? 0 : 1);  // activations 2, payload, Q8_0 scales
    static constexpr int ACT = 0;                      // 128 tokens x 64 B (folded fp16), swizzled 16-token groups
    static constexpr int WQ = ACT + MMA_TOK * 64;      // [wave][64 rows][PAY]
    static constexpr int WD = WQ + 4 * 64 * PAY;       // (Q8_0) [wave][64 rows] fp16 in the low half of a dword
    static constexpr int BYTES = WD + (SG ? 0 : 4 * 64 * 4);
    static constexpr int SR = MMA_RING * BYTES;        // (Q4_0) scale ring [2 groups][4 waves][64 rows][8 fp16]
    static constexpr int LDS = SR + (SG ? 2 * 4 * 1024 : 0);
    static_assert(LDS >= 4 * 32 * 68 * 4, "the epilogue's transpose fits the ring");
};

template <int TYPE, int NJ>
__device__ __forceinline__ void coop_tile(const MmaArgs& g, const Tile& tl, int cnt, unsigned char* ring, int bx)
{
    using SL = CoopSlot<TYPE>;
    constexpr int PAY = SL::PAY;
    const int tid = threadIdx.x, lane = tid & 63, r32 = lane & 31, h = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gI = bx * 4 + wave;
    const bool live = gI < g.rg;  // a wave past the last row group loads its share and multiplies nothing
    const int nb = g.nb;
    const uint32_t ring0 = (uint32_t)(uintptr_t)(lds_void_t)ring;

    const bool lst = g.npos > 0;
    const uint32_t xstep = lst ? (uint32_t)g.npos * 64u : 64u;  // bytes per block
    // activation rows of tokens 32 w + 16 i + lane / 4, part (lane % 4) ^ (lane / 16)
    uint32_t vx[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int t = min(32 * wave + 16 * i + (lane >> 2), cnt - 1);  // past cnt: a valid row, never stored
        const int q = (lane & 3) ^ ((lane >> 4) & 3);
        const int64_t row = lst ? (int64_t)(tl.start + t) * 32 : (int64_t)(g.perm[tl.start + t] / g.act_div) * g.act.qhstride;
        vx[i] = (uint32_t)(2 * (row + 8 * q));
    }
    const int gIc = min(gI, g.rg - 1);
    const __amdgpu_buffer_rsrc_t r_act = buf_rsrc(g.act.qh);
    const __amdgpu_buffer_rsrc_t r_w = buf_rsrc(g.payload + tl.e * g.mat_pay + gIc * g.rg_pay);
    const uint32_t vwq = 16 * lane;                           // payload: the row group's block, 1 KB per load
    const uint32_t vwd = (uint32_t)g.sc_off + 16 * lane;      // scales of row `lane`: (b / 8, row) * 16 + (b % 8) * 2

    auto issue = [&](auto SC, int b) {
        constexpr int S = decltype(SC)::value;
        const uint32_t bc = (uint32_t)min(b, nb - 1);
        unsigned char* slot = ring + S * SL::BYTES;
        const uint32_t sx = bc * xstep;
        if constexpr (SL::SG) {
            if ((b & 7) == 0)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(r_w, (lds_void_t)(ring + SL::SR + ((b >> 3) & 1) * 4096 + 1024 * wave),
                                                         16, vwd, (uint32_t)min(b >> 3, (nb - 1) >> 3) * 1024, 0, 0);
        }
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r_act, (lds_void_t)(slot + SL::ACT + (2 * wave) * 1024), 16, vx[0], sx, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r_act, (lds_void_t)(slot + SL::ACT + (2 * wave + 1) * 1024), 16, vx[1], sx,
                                                 0, 0);
        if constexpr (!SL::SG)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r_w, (lds_void_t)(slot + SL::WD + 256 * wave), 2, vwd,
                                                     (bc >> 3) * 1024 + (bc & 7) * 2, 0, 0);
#pragma unroll
        for (int i = 0; i < SL::WL; i++)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(r_w, (lds_void_t)(slot + SL::WQ + 64 * PAY * wave + 1024 * i), 16, vwq,
                                                     bc * 64 * PAY + 1024 * i, 0, 0);
    };
    auto land = [&](auto SC, int b) {  // S = b % MMA_RING (see mma_tile)
        constexpr int S = decltype(SC)::value;
        __builtin_amdgcn_s_waitcnt((SL::DMA * (MMA_RING - 2)) | (0x7 << 4) | (0xF << 8));
        __builtin_amdgcn_s_barrier();
        issue(ic<(S + MMA_RING - 1) % MMA_RING>{}, b + MMA_RING - 1);
    };

    mf16 C[2][NJ];
#pragma unroll
    for (int t = 0; t < 2; t++)
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int q = 0; q < 16; q++) C[t][j][q] = 0.0f;

    static_assert(3 * SL::BYTES + 3 * 2048 + 1024 + 64 < 65536, "ring offsets fit the LDS immediate");
    // lane (r32, h) of tile t: row 32 t + r32 of the wave's row group, k values 8 h .. 8 h + 7 (A0) and
    // 16 + 8 h .. (A1); the activations as in mma_tile
    const uint32_t A_WQ = ring0 + SL::WQ + 64 * PAY * wave + PAY * r32 + 8 * h;
    const uint32_t A_SG = ring0 + SL::SR + 1024 * wave + 16 * r32;
    const uint32_t A_WD = ring0 + SL::WD + 256 * wave + 4 * r32;
    const uint32_t A_B0 = ring0 + SL::ACT + act_off(r32, h), A_B1 = ring0 + SL::ACT + act_off(r32, 2 + h);

    // a block's operands as read from LDS, in two register sets (block b in set b % 2, so the next block's
    // reads land beside the operands being multiplied); valid after `landed`, in the reads' basic block
    u32x2 q[2][2][SL::WL];
    uint32_t wd[2][2];
    u32x4 fb0[2][NJ], fb1[2][NJ];
    auto reads = [&](auto SC, int b) {  // block b in slot S, into set S % 2
        constexpr int S = decltype(SC)::value, O = S * SL::BYTES, s = S & 1;
        q[s][0][0] = ds_r64<O>(A_WQ);
        q[s][1][0] = ds_r64<O + 32 * PAY>(A_WQ);
        if constexpr (PAY == 32) {
            q[s][0][SL::WL - 1] = ds_r64<O + 16>(A_WQ);
            q[s][1][SL::WL - 1] = ds_r64<O + 32 * PAY + 16>(A_WQ);
        }
        if constexpr (SL::SG) {
            const uint32_t a = A_SG + (uint32_t)(((b >> 3) & 1) * 4096 + (b & 7) * 2);
            wd[s][0] = ds_ru16<0>(a);
            wd[s][1] = ds_ru16<512>(a);
        } else {
            wd[s][0] = ds_ru16<O>(A_WD);
            wd[s][1] = ds_ru16<O + 128>(A_WD);
        }
        static_for<NJ>([&](auto JC) {
            constexpr int j = decltype(JC)::value;
            fb0[s][j] = ds_r128<O + 2048 * j>(A_B0);
            fb1[s][j] = ds_r128<O + 2048 * j>(A_B1);
        });
    };
    auto landed = [&](auto SC) {  // set S % 2
        constexpr int s = decltype(SC)::value & 1;
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int t = 0; t < 2; t++) {
#pragma unroll
            for (int i = 0; i < SL::WL; i++) tie(q[s][t][i]);
            tie(wd[s][t]);
        }
        static_for<NJ>([&](auto JC) {
            constexpr int j = decltype(JC)::value;
            tie(fb0[s][j]);
            tie(fb1[s][j]);
        });
    };
    // weight operand (tile t, k-half kh) of the block in set s: (q - 8) * d_w (Q4_0) or q * d_w (Q8_0) in fp16
    auto fold_w = [&](int s, int t, int kh) -> mh8 {
        const _Float16 dw = __builtin_bit_cast(_Float16, (uint16_t)wd[s][t]);
        const mh8 dw8 = {dw, dw, dw, dw, dw, dw, dw, dw};
        if (TYPE == PHX_Q4_0_DEV) {
            const u32x2 w = q[s][t][0];
            return kh ? bias8((w.x >> 4) & 0x0F0F0F0Fu, (w.y >> 4) & 0x0F0F0F0Fu, 1032.0f) * dw8
                      : bias8(w.x & 0x0F0F0F0Fu, w.y & 0x0F0F0F0Fu, 1032.0f) * dw8;
        } else {
            const u32x2 w = q[s][t][kh ? SL::WL - 1 : 0];
            return bias8(w.x ^ 0x80808080u, w.y ^ 0x80808080u, 1152.0f) * dw8;
        }
    };

    // block b (slot S, its operands landed in set S % 2): land block b + 1 and issue its reads into the
    // other set, then this block's products: each weight operand is folded just before the NJ MFMAs that
    // take it, the next operand's fold interleaved with them, so the wave's VALU runs beside its own
    // matrix-core work; the reads' wait closes the block (after the last block: a harmless extra barrier
    // and reads of a slot nobody uses)
    auto block = [&](auto SC, int b) {
        constexpr int S = decltype(SC)::value, s = S & 1, S1 = (S + 1) % MMA_RING;
        land(ic<S1>{}, b + 1);
        if (live) {  // uniform
            reads(ic<S1>{}, b + 1);
            __builtin_amdgcn_sched_barrier(0);
            // operand order (t, kh) = (0, 0), (1, 0), (0, 1), (1, 1): an accumulator's two products are
            // 2 NJ MFMAs apart
            mh8 A = fold_w(s, 0, 0);
            static_for<4>([&](auto UC) {
                constexpr int u = decltype(UC)::value, t = u & 1, kh = u >> 1;
                mh8 An = A;
                if constexpr (u < 3) An = fold_w(s, (u + 1) & 1, (u + 1) >> 1);
                static_for<NJ>([&](auto JC) {
                    constexpr int j = decltype(JC)::value;
                    C[t][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A, __builtin_bit_cast(mh8, kh ? fb1[s][j] : fb0[s][j]),
                                                                     C[t][j], 0, 0, 0);
                });
                if constexpr (u < 3) {
                    // the next operand's fold beside these MFMAs: one MFMA, then a few VALU, in turn
                    static_for<NJ>([&](auto) {
                        __builtin_amdgcn_sched_group_barrier(0x008, 1, u);
                        __builtin_amdgcn_sched_group_barrier(0x002, 4, u);
                    });
                }
                A = An;
            });
            __builtin_amdgcn_sched_barrier(0);
            landed(ic<S1>{});  // in the reads' basic block: the loop carries landed values
        }
        __builtin_amdgcn_sched_barrier(0);
    };

    issue(ic<0>{}, 0);
    issue(ic<1>{}, 1);
    issue(ic<2>{}, 2);
    static_assert(MMA_RING == 4, "the block loop is unrolled by the ring size");
    land(ic<0>{}, 0);
    if (live) {
        reads(ic<0>{}, 0);
        landed(ic<0>{});
    }
    for (int b = 0; b < nb; b += 4) {
        block(ic<0>{}, b);
        if (b + 1 < nb) block(ic<1>{}, b + 1);
        if (b + 2 < nb) block(ic<2>{}, b + 2);
        if (b + 3 < nb) block(ic<3>{}, b + 3);
    }
    // the loads issued past the last block land in this workgroup's LDS: let them finish, and every wave
    // be done with the ring, before the epilogue reuses it
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (!live) return;

    // lane (r32, h) holds, for token column r32 of tile j, rows 8 (q / 4) + 4 h + q % 4 of each half
    if (g.qout.qh) {  // uniform: the GELU-gated Q8_0 requant of the down input (src/GemmaCpu.cs:415, src/CpuRef.cs:49-62)
        float tv[NJ][16];
#pragma unroll
        for (int j = 0; j < NJ; j++)
#pragma unroll
            for (int q = 0; q < 16; q++) tv[j][q] = g.gelu_tab[f2h_bits(C[0][j][q])];
        const Act& o = g.qout;
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            float e[16], am = 0.0f;
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const float v = C[0][j][q];
                const float gl = v <= -10.0f ? 0.0f : (v >= 10.0f ? v : tv[j][q]);
                const int col = gI * 32 + 8 * (q >> 2) + 4 * h + (q & 3);
                e[q] = col < g.split ? gl * C[1][j][q] : 0.0f;
                am = fmaxf(am, fabsf(e[q]));
            }
            am = fmaxf(am, __shfl_xor(am, 32, 64));  // the other 16 columns: lane r32 + 32 (1 - 2 h)
            const float dd = am / 127.0f;
            const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
            const float dv = h2f(f2h_bits(dd));  // the block's fp16 scale
            uint32_t w[4][2];
#pragma unroll
            for (int g4 = 0; g4 < 4; g4++) {
                const int q0 = (int)roundf(e[4 * g4] * id), q1 = (int)roundf(e[4 * g4 + 1] * id),
                          q2 = (int)roundf(e[4 * g4 + 2] * id), q3 = (int)roundf(e[4 * g4 + 3] * id);
                w[g4][0] = fold_pair(q0, q1, dv);  // the down product's operands, folded
                w[g4][1] = fold_pair(q2, q3, dv);
            }
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

    if (g.paired && !g.out0) return;  // no g and u outputs: the requant above was the product's output
    const bool vec = (g.out_stride & 3) == 0;
    if (!g.paired) {
        // rows of a token through LDS: each 16-lane group then stores 256 contiguous bytes of one output
        // row (whole cache lines) instead of 32 lanes storing 32-byte pieces of 32 rows
        float* tb = (float*)ring + wave * (32 * 68);  // [32 tokens][64 rows + 4 pad]
        const int c16 = lane & 15, row0 = gI * 64 + 4 * c16;
        const bool full = vec && row0 + 3 < min(g.rows, g.split);
        // the tile's assignment indices (32 NJ <= 128): lane l loads positions l and 64 + l before any
        // store, a store round takes its own by a lane shuffle (a load per round would wait behind the
        // previous round's stores)
        static_assert(NJ <= 4, "two indices per lane cover the tile");
        const int pa0 = g.perm[tl.start + min(lane, cnt - 1)], pa1 = g.perm[tl.start + min(64 + lane, cnt - 1)];
#pragma unroll
        for (int j = 0; j < NJ; j++) {
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int q4 = 0; q4 < 4; q4++)
                    *(float4*)(tb + r32 * 68 + 32 * t + 8 * q4 + 4 * h) =
                        make_float4(C[t][j][4 * q4], C[t][j][4 * q4 + 1], C[t][j][4 * q4 + 2], C[t][j][4 * q4 + 3]);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
            for (int rd = 0; rd < 8; rd++) {
                const int tok = 4 * rd + (lane >> 4), sidx = 32 * j + tok;
                const float4 v = *(const float4*)(tb + tok * 68 + 4 * c16);
                const int av = __shfl(j < 2 ? pa0 : pa1, 32 * (j & 1) + tok, 64);
                if (sidx < cnt) {
                    const int64_t a = av;
                    if (full) *(float4*)(g.out0 + a * g.out_stride + row0) = v;
                    else {
                        const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const int r = row0 + i;
                            if (r < g.rows) {
                                if (r < g.split) g.out0[a * g.out_stride + r] = vv[i];
                                else g.out1[a * g.out_stride + r - g.split] = vv[i];
                            }
                        }
                    }
                }
            }
            // every lane's reads of this tile end before the next tile's writes
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        }
        return;
    }
    int pa[NJ];  // every index load before the first store
#pragma unroll
    for (int j = 0; j < NJ; j++) pa[j] = g.perm[tl.start + min(32 * j + r32, cnt - 1)];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int sidx = 32 * j + r32;
        if (sidx >= cnt) continue;
        const int64_t a = pa[j];
#pragma unroll
        for (int half = 0; half < 2; half++)
#pragma unroll
            for (int q4 = 0; q4 < 4; q4++) {
                const int lg0 = half * 32 + 8 * q4 + 4 * h;  // lane within the row group of the first of four
                const float4 v = make_float4(C[half][j][4 * q4], C[half][j][4 * q4 + 1], C[half][j][4 * q4 + 2],
                                             C[half][j][4 * q4 + 3]);
                if (g.paired) {
                    const int col = gI * 32 + (lg0 & 31);
                    float* dst = (half ? g.out1 : g.out0) + a * g.out_stride + col;
                    if (vec && col + 3 < g.split) *(float4*)dst = v;
                    else
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            if (col + i < g.split) dst[i] = C[half][j][4 * q4 + i];
                } else {
                    const int row = gI * 64 + lg0;
                    if (vec && row + 3 < min(g.rows, g.split)) *(float4*)(g.out0 + a * g.out_stride + row) = v;
                    else
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const int r = row + i;
                            if (r < g.rows) {
                                if (r < g.split) g.out0[a * g.out_stride + r] = C[half][j][4 * q4 + i];
                                else g.out1[a * g.out_stride + r - g.split] = C[half][j][4 * q4 + i];
                            }
                        }
                }
            }
    }
}

template <int TYPE>
__global__ __launch_bounds__(256, 2) void k_grouped_coop(MmaArgs g)
{
    __shared__ __align__(16) unsigned char ring[CoopSlot<TYPE>::LDS];
    int bx;
    const int tile = xcd_tile(&bx);
    if (tile >= *g.ntiles) return;  // uniform over the workgroup
    const Tile tl = g.tiles[tile];
    const int cnt = min(tl.cnt, MMA_TOK);
#ifdef PHX_TIMELINE
    const int wgf = tile * gridDim.x + bx, tbase = g.paired ? 0 : 16384;  // as in k_grouped_mfma
    if (threadIdx.x == 0 && wgf < 8192) phx_tl[tbase + 2 * wgf] = wall_clock64();
#endif
    switch ((cnt + 31) / 32) {  // active 32-token column tiles
    case 1: coop_tile<TYPE, 1>(g, tl, cnt, ring, bx); break;
    case 2: coop_tile<TYPE, 2>(g, tl, cnt, ring, bx); break;
    case 3: coop_tile<TYPE, 3>(g, tl, cnt, ring, bx); break;
    default: coop_tile<TYPE, 4>(g, tl, cnt, ring, bx); break;
    }
#ifdef PHX_TIMELINE
    if (threadIdx.x == 0 && wgf < 8192) phx_tl[tbase + 2 * wgf + 1] = wall_clock64();
#endif
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
    if (act.fold) {  // the tolerance mode's folded operands (its gate|up writes the down input folded too)
        const dim3 grid((w.rg + 3) / 4, xcd_tile_slots(max_tiles));
        if (w.type == PHX_Q4_0_DEV) launch(k_grouped_coop<PHX_Q4_0_DEV>, grid, dim3(256), 0, st, g);
        else launch(k_grouped_coop<PHX_Q8_0_DEV>, grid, dim3(256), 0, st, g);
        return;
    }
    const dim3 grid((w.rg + 1) / 2, xcd_tile_slots(max_tiles));
    if (w.type == PHX_Q4_0_DEV) launch(k_grouped_mfma<PHX_Q4_0_DEV>, grid, dim3(256), 0, st, g);
    else launch(k_grouped_mfma<PHX_Q8_0_DEV>, grid, dim3(256), 0, st, g);
}

// ============================================================================ K-quant products
// DotK (src/CpuRefKQuants.cs:177-212) per (row, assignment): per 256-element super-block the eight
// integer lanes aux32[l] = sum over the 32 elements e = 8 i + l of scale(e) * a(e) * x(e), the float
// lanes sums[l] += (d * yd) * aux32[l], for Q4_K the min term sumf -= (dmin * yd) * sumi with
// sumi = sum_j bsum_j * min(j / 2); after the last super-block sumf += sums[l] in l order.
// Per super-block and 16 x 16 (row, assignment) tile on the matrix cores:
//   - aux32[l] is one v_mfma_f32_16x16x32_f16 over lane l's 32 elements: the weights enter as
//     scale * a, the activations as their Q8_K integers, all exact in fp16 (Q4_K: scale * a <= 945),
//     and every partial sum is an integer of magnitude at most 2^24, exact in fp32 in any order.
//     Q6_K's scale * a reaches 4096, past fp16's exact odd integers: with scale = 32 hi + lo
//     (lo = 0..31) it enters as lo * a (|.| <= 992) and 32 hi * a (a multiple of 32, |.| <= 4096),
//     two products into one accumulator;
//   - sumi is one v_mfma_f32_16x16x16_f16 of the mins against the fp16 block sums (|bsum| <= 2048);
//   - the float chain runs on VALU in the reference's order, so results equal DotK bit for bit.
// Operand layouts (gfx950): v_mfma_f32_16x16x32_f16 A lane l holds row l % 16 and k = 8 (l / 16) + e,
// e = 0..7, B lane l column l % 16 and the same k, and the 16 x 16 result D[i][j] sits in lane
// j + 16 (i / 4), register i % 4; v_mfma_f32_16x16x16_f16 the same with k = 4 (l / 16) + e, e = 0..3.
// Lane quarter q's k = 8 q + e is element 32 s + l + 8 mm of the super-block with s = 2 q + e / 4 and
// mm = {0, 2, 1, 3}[e % 4]: the activations' fp16 copy holds, per row and super-block, the halves
// [l][s][mm'] (x(32 s + l + 8 {0, 2, 1, 3}[mm'])), so a quarter's eight values are the 16-byte chunk
// 4 l + q, and the repacked weights (bytes (s, l / 2, mm): low nibble l even, high nibble l odd) give
// the pairs (mm 0, 2) and (mm 1, 3) of a byte-lane dword by one mask each.
//
// Work layout: a workgroup of eight waves covers two row groups (wave w: rows 16 (w % 4) .. + 15 of
// row group 2 x + w / 4) and one tile of up to 48 assignments (three 16-assignment column tiles).  Per
// super-block its operands reach LDS by direct loads into a ring slot, RING - 1 super-blocks ahead: the
// activation chunks chunk-major ([chunk][assignment][16 B]: the 16 lanes of an operand read one
// 256-byte run), Q4_K block sums and token scales, each wave's 16 weight rows and their scales.  Each
// wave issues the same KM_DMA loads per super-block (some with lanes masked off), so its own count of
// outstanding loads tells when a super-block has landed.
constexpr int KM_TOK = 48;  // assignments per tile (kKmmaTile)
static_assert(KM_TOK == kKmmaTile, "tile capacity");
constexpr int KM_NW = 8;    // waves per workgroup
constexpr int KM_DMA = 9;   // direct loads per wave per super-block
constexpr int KM_RING = 3;  // ring slots

// LDS ring, region-major: each region holds its KM_RING slots one after another, so a lane's read
// address in a region is one VGPR and the slot an immediate offset
template <int TYPE>
struct KmRing {
    static constexpr bool Q4K = TYPE == PHX_Q4_K_DEV;
    static constexpr int PAY = Q4K ? 144 : 208;
    static constexpr int ACT_N = 32 * KM_TOK * 16;          // [32 chunks][48 assignments][16 B]
    static constexpr int BSM_N = Q4K ? 4 * KM_TOK * 8 : 0;  // Q4_K: [4 quarters][48][4 fp16 bsums]
    static constexpr int YD_N = KM_TOK * 4;                 // [48] token scales
    static constexpr int W_N = KM_NW * 16 * PAY;            // [8 waves][16 rows][PAY]
    static constexpr int WS_N = KM_NW * 16 * 4;             // [8 waves][16 rows] 4-byte slots
    static constexpr int ACT = 0, BSM = ACT + KM_RING * ACT_N, YD = BSM + KM_RING * BSM_N;
    static constexpr int W = YD + KM_RING * YD_N, WS = W + KM_RING * W_N, BYTES = WS + KM_RING * WS_N;
    static_assert(W % 16 == 0 && WS % 16 == 0, "16-byte direct loads land aligned");
};

typedef _Float16 mh4 __attribute__((ext_vector_type(4)));
typedef float mf4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t pk_fma(uint32_t a, mh2 b, mh2 c)
{
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(mh2, a), b, c));
}
__device__ __forceinline__ mh2 hpair(_Float16 a, _Float16 b) { return mh2{a, b}; }
// (x & m) | c in one instruction (the compiler splits it to keep the constants out of SGPRs)
__device__ __forceinline__ uint32_t and_or(uint32_t x, uint32_t m, uint32_t c)
{
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(m), "v"(c));  // one SGPR operand (gfx9)
    return r;
}

// FOLD (the tolerance mode, PHX_FLAG_FAST_MATH): the activations arrive folded (fp16(q * d) of their
// Q8_K scale), each weight operand is folded per super-block, fp16(sc * q * d - dmin * m) for Q4_K (one
// rounding, dmin * m first rounded to fp16) and fp16(lo * q * d), fp16(32 hi * q * d) for Q6_K's two
// parts, and every row accumulates over all its super-blocks in fp32 on the matrix cores: no per-lane
// float chain, no min term, no scale products.
template <int TYPE, int NJ, bool FOLD>
__device__ __forceinline__ void kmma_tile(const MmaArgs& g, const Tile& tl, int cnt, unsigned char* ring, int bx)
{
    using RG = KmRing<TYPE>;
    constexpr bool Q4K = RG::Q4K;
    constexpr int PAY = RG::PAY, RING = KM_RING, SBY = Q4K ? 4 : 2;
    const int tid = threadIdx.x, lane = tid & 63, r16 = lane & 15, q = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int gI = bx * 2 + (wave >> 2), ws = wave & 3;
    const bool live = gI < g.rg;  // a wave past the last row group computes a clamped one, stores nothing
    const int nb = g.nb;
    const uint32_t ring0 = (uint32_t)(uintptr_t)(lds_void_t)ring;

    // the direct loads' lane sources (assignments past cnt: a valid row, never stored), as buffer -> LDS
    // loads: each lane's byte offset (a VGPR, the same for every super-block) and the super-block's
    // uniform offset (an SGPR)
    auto arow = [&](int t) -> int64_t { return g.perm[tl.start + min(t, cnt - 1)] / g.act_div; };
    // (1)-(3) activation chunks: load i of wave w fills positions 64 (3 w + i) + lane of the
    // [chunk][assignment] array: chunk p / 48 of assignment p % 48
    uint32_t vx[3];
#pragma unroll
    for (int i = 0; i < 3; i++) {
        const int p = 64 * (3 * wave + i) + lane;
        vx[i] = (uint32_t)(2 * (arow(p % KM_TOK) * g.act.qhstride + 8 * (p / KM_TOK)));
    }
    // (4) Q4_K: dword 48 w + lane (lanes 0-47) of the block sums' [quarter][assignment][2 dwords]
    uint32_t vb = 0;
    if (Q4K) {
        const int dw = 48 * wave + min(lane, 47);
        vb = (uint32_t)(2 * (arow((dw % 96) >> 1) * g.act.bhstride + 4 * (dw / 96) + 2 * (dw & 1)));
    }
    // (5) token scales of assignments 6 w + lane (lanes 0-5)
    const uint32_t vy = (uint32_t)(4 * arow(6 * wave + min(lane, 5)) * g.act.dstride);
    // (6)-(8) the wave's 16 weight rows, 1 KB per load; (9) their scales (lanes 0-15)
    const int gIc = min(gI, g.rg - 1);
    const __amdgpu_buffer_rsrc_t r_act = buf_rsrc(g.act.qh), r_yd = buf_rsrc(g.act.d);
    const __amdgpu_buffer_rsrc_t r_bh = buf_rsrc(Q4K ? (const void*)g.act.bh : (const void*)g.act.d);
    const __amdgpu_buffer_rsrc_t r_w = buf_rsrc(g.payload + tl.e * g.mat_pay + gIc * g.rg_pay);
    const __amdgpu_buffer_rsrc_t r_s = buf_rsrc(g.scale + tl.e * g.mat_sc + (int64_t)gIc * nb * 64 * SBY);
    const uint32_t vw = 16 * ws * PAY + 16 * lane, vs = (16 * ws + r16) * SBY;

#define KM_LOAD(rsrc, lds_off, size, voff, soff) \
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t)(ring + (lds_off)), size, voff, soff, 0, 0)
    auto issue = [&](auto SC, int b) {  // super-block b (clamped: past the end a harmless reload) into slot S
        constexpr int S = decltype(SC)::value;
        const uint32_t bc = (uint32_t)min(b, nb - 1);
        const uint32_t sw = bc * 64 * PAY;
        const int wl = RG::W + S * RG::W_N + wave * 16 * PAY;
#pragma unroll
        for (int i = 0; i < 3; i++) KM_LOAD(r_act, RG::ACT + S * RG::ACT_N + (3 * wave + i) * 1024, 16, vx[i], bc * 512);
        if (Q4K) {
            if (lane < 48) KM_LOAD(r_bh, RG::BSM + S * RG::BSM_N + 192 * wave, 4, vb, bc * 32);
        } else {
            if (lane < 16) KM_LOAD(r_w, wl + 3072, 16, vw, sw + 3072);  // Q6_K rows: 3328 bytes
        }
        if (lane < 6) KM_LOAD(r_yd, RG::YD + S * RG::YD_N + 24 * wave, 4, vy, bc * 4);
        KM_LOAD(r_w, wl, 16, vw, sw);
        KM_LOAD(r_w, wl + 1024, 16, vw, sw + 1024);
        if (Q4K) {
            if (lane < 16) KM_LOAD(r_w, wl + 2048, 16, vw, sw + 2048);  // Q4_K rows: 2304 bytes
        } else {
            KM_LOAD(r_w, wl + 2048, 16, vw, sw + 2048);
        }
        if (lane < 16) {
            if (Q4K) KM_LOAD(r_s, RG::WS + S * RG::WS_N + 64 * wave, 4, vs, bc * 64 * SBY);
            else KM_LOAD(r_s, RG::WS + S * RG::WS_N + 64 * wave, 2, vs, bc * 64 * SBY);
        }
    };
#undef KM_LOAD
    // super-block b (slot S) has landed once at most the later ones' loads are outstanding; the barrier
    // then publishes it and ends every wave's reads of the slot that issue(b + RING - 1) refills
    auto land = [&](auto SC, int b) {
        constexpr int S = decltype(SC)::value;
        __builtin_amdgcn_s_waitcnt(vm_wait(KM_DMA * (RING - 2)));
        __builtin_amdgcn_s_barrier();
        issue(ic<(S + RING - 1) % RING>{}, b + RING - 1);
    };

    float sums[8][NJ][4], sumf[NJ][4];
#pragma unroll
    for (int c = 0; c < NJ; c++)
#pragma unroll
        for (int v = 0; v < 4; v++) {
            sumf[c][v] = 0.0f;
#pragma unroll
            for (int l = 0; l < 8; l++) sums[l][c][v] = 0.0f;
        }
    const mf4 zero4 = {};
    mf4 acc[NJ];  // FOLD: the tiles' fp32 sums over all super-blocks
#pragma unroll
    for (int c = 0; c < NJ; c++) acc[c] = zero4;
    // the lane's LDS read addresses in slot 0 of each region (slot S: + S * region slot bytes in the
    // immediate; the third activation slot from a second address, past the immediate's 64 KB)
    const uint32_t a_act = ring0 + RG::ACT + q * (KM_TOK * 16) + r16 * 16, a_act2 = a_act + 2 * RG::ACT_N;
    const uint32_t a_bs = ring0 + RG::BSM + q * (KM_TOK * 8) + r16 * 8;
    const uint32_t a_yd = ring0 + RG::YD + r16 * 4;
    const uint32_t a_row = ring0 + RG::W + (wave * 16 + r16) * PAY + 32 * q;
    const uint32_t a_sc = ring0 + RG::W + (wave * 16 + r16) * PAY + (Q4K ? 128 + 4 * (q >> 1) : 128 + 16 * q);
    const uint32_t a_y = Q4K ? a_sc + 8 : ring0 + RG::W + (wave * 16 + r16) * PAY + 192 + 4 * q;
    const uint32_t a_ws = ring0 + RG::WS + (wave * 16 + 4 * q) * 4;
    const uint32_t a_wr = ring0 + RG::WS + (wave * 16 + r16) * 4;  // FOLD: d (and dmin) of the A operand's row
    static_assert((RING - 1) * RG::W_N + 192 + 16 * 3 + 16 < 65536, "weight slots within the LDS immediate");
    static_assert(RG::ACT_N + 8 * KM_TOK * 64 < 65536, "two activation slots within the LDS immediate");
    // activation chunk reads of slot S at inner offset O
    auto act_rd = [&](auto SC, auto OC) -> u32x4 {
        constexpr int S = decltype(SC)::value, O = decltype(OC)::value;
        if constexpr (S < 2) return ds_r128<S * RG::ACT_N + O>(a_act);
        else return ds_r128<(S - 2) * RG::ACT_N + O>(a_act2);
    };

    // super-block b in slot S
    auto sblock = [&](auto SC, int b) {
        constexpr int S = decltype(SC)::value;
        land(SC, b);
        // the super-block's weights, row scales, token scales, block sums and the first operands (a read's
        // result is used only after its wait, never first composed into another value)
        constexpr int OW = S * RG::W_N;
        u32x4 D0 = ds_r128<OW>(a_row), D1 = ds_r128<OW + 16>(a_row);
        // Q4_K: X0 the dword of sc[2 q], sc[2 q + 1], Y that of mins[2 q], mins[2 q + 1];
        // Q6_K: X the high-bit dwords (s = 2 q: lq 0, 1; s = 2 q + 1: lq 0, 1), Y sc[4 q .. 4 q + 3]
        u32x4 X;
        uint32_t X0;
        if (Q4K) X0 = ds_r32<OW>(a_sc);
        else X = ds_r128<OW>(a_sc);
        uint32_t Y = ds_r32<OW>(a_y);
        u32x4 WSV = {0u, 0u, 0u, 0u};
        uint32_t WR = 0;
        if constexpr (FOLD) WR = ds_r32<S * RG::WS_N>(a_wr);
        else WSV = ds_r128<S * RG::WS_N>(a_ws);
        uint32_t YD[NJ];
        u32x2 BS[NJ];
        u32x4 B[2][NJ];
        constexpr int OY = S * RG::YD_N, OB = S * RG::BSM_N;
        if (!FOLD) YD[0] = ds_r32<OY>(a_yd);
        if (Q4K && !FOLD) BS[0] = ds_r64<OB>(a_bs);
        B[0][0] = act_rd(SC, ic<0>{});
        if (NJ > 1) {
            if (!FOLD) YD[1 % NJ] = ds_r32<OY + 64>(a_yd);
            if (Q4K && !FOLD) BS[1 % NJ] = ds_r64<OB + 128>(a_bs);
            B[0][1 % NJ] = act_rd(SC, ic<256>{});
        }
        if (NJ > 2) {
            if (!FOLD) YD[2 % NJ] = ds_r32<OY + 128>(a_yd);
            if (Q4K && !FOLD) BS[2 % NJ] = ds_r64<OB + 256>(a_bs);
            B[0][2 % NJ] = act_rd(SC, ic<512>{});
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        tie(D0);
        tie(D1);
        if (Q4K) tie(X0);
        else tie(X);
        tie(Y);
        if constexpr (FOLD) tie(WR);
        else tie(WSV);
#pragma unroll
        for (int c = 0; c < NJ; c++) {
            if (!FOLD) tie(YD[c]);
            if (Q4K && !FOLD) tie(BS[c]);
            tie(B[0][c]);
        }
        // d * yd (and dmin * yd) per (row 4 q + v, assignment)
        float dd[NJ][4], dm[NJ][4];
        if constexpr (!FOLD) {
#pragma unroll
            for (int c = 0; c < NJ; c++)
#pragma unroll
                for (int v = 0; v < 4; v++) {
                    const float yd = __uint_as_float(YD[c]);
                    dd[c][v] = h2f(WSV[v] & 0xFFFFu) * yd;
                    if (Q4K) dm[c][v] = h2f(WSV[v] >> 16) * yd;
                }
        }
        // FOLD: the row's d as an fp16 pair and, for Q4_K, -fp16(dmin * m) of sub-blocks 2 q, 2 q + 1
        const _Float16 dwh = __builtin_bit_cast(_Float16, (uint16_t)(WR & 0xFFFFu));
        const mh2 D2 = hpair(dwh, dwh);
        mh2 MT[2];
        if (FOLD && Q4K) {
            const uint32_t mw = Y >> (16 * (q & 1));  // mins[2 q], mins[2 q + 1]
            const float dmin = h2f(WR >> 16);
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const _Float16 mt = (_Float16)(dmin * (float)(int)((mw >> (8 * j)) & 0xFFu));  // exact, then rounded once
                MT[j] = hpair(-mt, -mt);
            }
        }
        // per-s constants of the A operands (s = 2 q, 2 q + 1).  Q4_K: the nibble n enters as the half
        // 1024 + n (l even) or 1024 + 16 n (l odd), so sc * n = fma(., sc, -1024 sc) or
        // fma(., sc / 16, -64 sc).  Q6_K: the 6-bit value v enters as 1024 + 4 v, q = v - 32, and with
        // sc = 32 hi + lo: lo * q = fma(., lo / 4, -288 lo), 32 hi * q = fma(., 8 hi, -9216 hi) (every
        // constant and result exact in fp16, each fma rounding once to an exact value)
        mh2 K0[2], M0[2], K1[2], M1[2];
        if (Q4K) {
            const uint32_t sw = X0 >> (16 * (q & 1));  // sc[2 q], sc[2 q + 1]
#pragma unroll
            for (int j = 0; j < 2; j++) {
                const _Float16 f = (_Float16)(int)((sw >> (8 * j)) & 0xFFu);
                K0[j] = hpair(f, f);
                M0[j] = hpair(f * (_Float16)-1024.0f, f * (_Float16)-1024.0f);
                K1[j] = hpair(f * (_Float16)0.0625f, f * (_Float16)0.0625f);
                M1[j] = hpair(f * (_Float16)-64.0f, f * (_Float16)-64.0f);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 2; j++) {  // sc[4 q + 2 j], sc[4 q + 2 j + 1]
                const int s0 = (int)(int8_t)(Y >> (16 * j)), s1 = (int)(int8_t)(Y >> (16 * j + 8));
                const _Float16 lo0 = (_Float16)(s0 & 31), lo1 = (_Float16)(s1 & 31);
                const _Float16 hi0 = (_Float16)(s0 >> 5), hi1 = (_Float16)(s1 >> 5);
                K0[j] = hpair(lo0 * (_Float16)0.25f, lo1 * (_Float16)0.25f);
                M0[j] = hpair(lo0 * (_Float16)-288.0f, lo1 * (_Float16)-288.0f);
                K1[j] = hpair(hi0 * (_Float16)8.0f, hi1 * (_Float16)8.0f);
                M1[j] = hpair(hi0 * (_Float16)-9216.0f, hi1 * (_Float16)-9216.0f);
            }
        }
        // lane l's A operand(s): pairs (s = 2 q: mm 0, 2), (mm 1, 3), then s = 2 q + 1
        auto a_op = [&](int l, mh8& A, mh8& A2) {
            const int p = l >> 1;
            const uint32_t x0 = D0[p], x1 = D1[p];
            uint32_t w[4];
            if (Q4K) {
                const uint32_t m = (l & 1) ? 0x00F000F0u : 0x000F000Fu;
                const mh2 k0 = (l & 1) ? K1[0] : K0[0], c0 = (l & 1) ? M1[0] : M0[0];
                const mh2 k1 = (l & 1) ? K1[1] : K0[1], c1 = (l & 1) ? M1[1] : M0[1];
                w[0] = pk_fma(and_or(x0, m, 0x64006400u), k0, c0);
                w[1] = pk_fma(and_or(x0 >> 8, m, 0x64006400u), k0, c0);
                w[2] = pk_fma(and_or(x1, m, 0x64006400u), k1, c1);
                w[3] = pk_fma(and_or(x1 >> 8, m, 0x64006400u), k1, c1);
                if constexpr (FOLD) {  // sc * q (exact) * d - fp16(dmin * m), one rounding
#pragma unroll
                    for (int i = 0; i < 4; i++) w[i] = pk_fma(w[i], D2, MT[i >> 1]);
                }
                A = __builtin_bit_cast(mh8, make_uint4(w[0], w[1], w[2], w[3]));
            } else {
                // the low nibble to bits 2-5 of each half, the two high bits (bits 2 i of the byte,
                // i = l % 4) to bits 6-7
                const int i = l & 3, lq = l >> 2;
                const uint32_t h0 = X[lq], h1 = X[2 + lq];
                auto lo = [&](uint32_t x, int pr) {
                    const int sh = ((l & 1) ? 4 : 0) + 8 * pr - 2;  // from bit sh + 2 to bit 2
                    return sh >= 0 ? x >> sh : x << -sh;
                };
                auto hi = [&](uint32_t h, int pr) {
                    const int sh = 2 * i + 8 * pr - 6;  // from bit sh + 6 to bit 6
                    return sh >= 0 ? h >> sh : h << -sh;
                };
                uint32_t v[4];
                v[0] = and_or(hi(h0, 0), 0x00C000C0u, and_or(lo(x0, 0), 0x003C003Cu, 0x64006400u));
                v[1] = and_or(hi(h0, 1), 0x00C000C0u, and_or(lo(x0, 1), 0x003C003Cu, 0x64006400u));
                v[2] = and_or(hi(h1, 0), 0x00C000C0u, and_or(lo(x1, 0), 0x003C003Cu, 0x64006400u));
                v[3] = and_or(hi(h1, 1), 0x00C000C0u, and_or(lo(x1, 1), 0x003C003Cu, 0x64006400u));
                uint32_t u[4];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    w[j] = pk_fma(v[j], K0[j >> 1], M0[j >> 1]);  // lo * (v - 32)
                    u[j] = pk_fma(v[j], K1[j >> 1], M1[j >> 1]);  // 32 hi * (v - 32)
                    if constexpr (FOLD) {  // each part times d, one rounding each
                        w[j] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(mh2, w[j]) * D2);
                        u[j] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(mh2, u[j]) * D2);
                    }
                }
                A = __builtin_bit_cast(mh8, make_uint4(w[0], w[1], w[2], w[3]));
                A2 = __builtin_bit_cast(mh8, make_uint4(u[0], u[1], u[2], u[3]));
            }
        };
        // lane l: operands of lane l + 1 read behind its products (immediate offsets: l compile-time)
        auto step = [&](auto LC) {
            constexpr int l = decltype(LC)::value, cur = l & 1;
            if (l + 1 < 8) {
                B[cur ^ 1][0] = act_rd(SC, ic<(l + 1) * KM_TOK * 64>{});
                if (NJ > 1) B[cur ^ 1][1 % NJ] = act_rd(SC, ic<(l + 1) * KM_TOK * 64 + 256>{});
                if (NJ > 2) B[cur ^ 1][2 % NJ] = act_rd(SC, ic<(l + 1) * KM_TOK * 64 + 512>{});
            }
            mh8 A, A2;
            a_op(l, A, A2);
#pragma unroll
            for (int c = 0; c < NJ; c++) {
                if constexpr (FOLD) {
                    acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, __builtin_bit_cast(mh8, B[cur][c]), acc[c], 0, 0, 0);
                    if (!Q4K)
                        acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A2, __builtin_bit_cast(mh8, B[cur][c]), acc[c], 0, 0, 0);
                } else {
                    mf4 C = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, __builtin_bit_cast(mh8, B[cur][c]), zero4, 0, 0, 0);
                    if (!Q4K) C = __builtin_amdgcn_mfma_f32_16x16x32_f16(A2, __builtin_bit_cast(mh8, B[cur][c]), C, 0, 0, 0);
                    // the reference chain: sums[l] += (d * yd) * aux32[l]
#pragma unroll
                    for (int v = 0; v < 4; v++) sums[l][c][v] = sums[l][c][v] + dd[c][v] * C[v];
                }
            }
            if (l + 1 < 8) {
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
                for (int c = 0; c < NJ; c++) tie(B[cur ^ 1][c]);
            }
        };
        step(ic<0>{});
        step(ic<1>{});
        step(ic<2>{});
        step(ic<3>{});
        step(ic<4>{});
        step(ic<5>{});
        step(ic<6>{});
        step(ic<7>{});
        if (Q4K && !FOLD) {  // the min term: sumf -= (dmin * yd) * sumi
            const uint32_t mw = Y >> (16 * (q & 1));  // mins[2 q], mins[2 q + 1]
            const _Float16 m0 = (_Float16)(int)(mw & 0xFFu), m1 = (_Float16)(int)((mw >> 8) & 0xFFu);
            const mh4 Am = {m0, m0, m1, m1};
#pragma unroll
            for (int c = 0; c < NJ; c++) {
                const mf4 Cm = __builtin_amdgcn_mfma_f32_16x16x16f16(Am, __builtin_bit_cast(mh4, BS[c]), zero4, 0, 0, 0);
#pragma unroll
                for (int v = 0; v < 4; v++) sumf[c][v] = sumf[c][v] - dm[c][v] * Cm[v];
            }
        }
    };

    issue(ic<0>{}, 0);
    issue(ic<1>{}, 1);
    // the ring's slots by unrolling: every LDS offset is an immediate
    static_assert(RING == 3, "the super-block loop is unrolled by the ring size");
    for (int b = 0; b < nb; b += 3) {
        sblock(ic<0>{}, b);
        if (b + 1 < nb) sblock(ic<1>{}, b + 1);
        if (b + 2 < nb) sblock(ic<2>{}, b + 2);
    }
    // the loads issued past the last super-block land in this workgroup's LDS: let them finish
    __builtin_amdgcn_s_waitcnt(0);
    if (!live) return;
    // lane (r16, q): assignment 16 c + r16, rows 4 q .. 4 q + 3 of the wave's 16; every index load
    // before the first store
    int pa[NJ];
#pragma unroll
    for (int c = 0; c < NJ; c++) pa[c] = g.perm[tl.start + min(16 * c + r16, cnt - 1)];
#pragma unroll
    for (int c = 0; c < NJ; c++) {
        const int t = 16 * c + r16;
        if (t >= cnt) continue;
        float o[4];
#pragma unroll
        for (int v = 0; v < 4; v++) {
            float s = sumf[c][v];
#pragma unroll
            for (int l = 0; l < 8; l++) s += sums[l][c][v];
            o[v] = FOLD ? acc[c][v] : s;
        }
        const int64_t a = pa[c];
        const int lg0 = 16 * ws + 4 * q;  // lane within the row group of the first of four
        const bool vec = (g.out_stride & 3) == 0;
        if (g.paired) {
            const int col = gI * 32 + (lg0 & 31);
            float* dst = (lg0 < 32 ? g.out0 : g.out1) + a * g.out_stride + col;
            if (vec && col + 3 < g.split) *(float4*)dst = make_float4(o[0], o[1], o[2], o[3]);
            else
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (col + i < g.split) dst[i] = o[i];
        } else {
            const int row = gI * 64 + lg0;
            if (vec && row + 3 < min(g.rows, g.split)) *(float4*)(g.out0 + a * g.out_stride + row) = make_float4(o[0], o[1], o[2], o[3]);
            else
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int r = row + i;
                    if (r < g.rows) {
                        if (r < g.split) g.out0[a * g.out_stride + r] = o[i];
                        else g.out1[a * g.out_stride + r - g.split] = o[i];
                    }
                }
        }
    }
}

template <int TYPE, bool FOLD>
__global__ __launch_bounds__(KM_NW * 64, 1) void k_grouped_kmma(MmaArgs g)
{
    extern __shared__ __align__(16) unsigned char kring[];
    // grid order (the XCD-aware order of the Q4_0 / Q8_0 kernel measured slower here: C4 gate|up
    // 227 -> 233 us, down 171 -> 175 us)
    const int bx = blockIdx.x, tile = blockIdx.y;
    if (tile >= *g.ntiles) return;  // uniform over the workgroup
    const Tile tl = g.tiles[tile];
    const int cnt = min(tl.cnt, KM_TOK);
    if (cnt > 32) kmma_tile<TYPE, 3, FOLD>(g, tl, cnt, kring, bx);
    else if (cnt > 16) kmma_tile<TYPE, 2, FOLD>(g, tl, cnt, kring, bx);
    else kmma_tile<TYPE, 1, FOLD>(g, tl, cnt, kring, bx);
}

void launch_grouped_kmma(hipStream_t st, const QMat& w, Act act, const Tile* tiles, const int* ntiles, int max_tiles,
                         const int* perm, int act_div, float* out0, float* out1, int split, int out_stride)
{
    MmaArgs g{};
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
    // the activations' format picks the arithmetic: folded fp16 copies take the tolerance mode
    auto go = [&](auto kern, size_t lds) {
        (void)hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        launch(kern, grid, dim3(KM_NW * 64), (uint32_t)lds, st, g);
    };
    if (w.type == PHX_Q4_K_DEV) {
        constexpr size_t lds = (size_t)KmRing<PHX_Q4_K_DEV>::BYTES;
        if (act.fold) go(k_grouped_kmma<PHX_Q4_K_DEV, true>, lds);
        else go(k_grouped_kmma<PHX_Q4_K_DEV, false>, lds);
    } else {
        constexpr size_t lds = (size_t)KmRing<PHX_Q6_K_DEV>::BYTES;
        if (act.fold) go(k_grouped_kmma<PHX_Q6_K_DEV, true>, lds);
        else go(k_grouped_kmma<PHX_Q6_K_DEV, false>, lds);
    }
}

}  // namespace phx

#ifdef PHX_TIMELINE
// the instrumented build's clock-stamp table of this file's kernels (as phxdbg_timeline)
extern "C" __attribute__((visibility("default"))) int phxdbg_timeline_prefill(unsigned long long* host, size_t n, int clear)
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
