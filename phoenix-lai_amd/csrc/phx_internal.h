// Internal types shared by the runtime (runtime.hip) and the gfx950 kernels (kernels.hip).
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "phx_moe.h"

#define PHX_Q4_0_DEV 2
#define PHX_Q8_0_DEV 8
#define PHX_Q4_K_DEV 12
#define PHX_Q5_K_DEV 13
#define PHX_Q6_K_DEV 14
#define PHX_IQ2_XXS_DEV 16
#define PHX_IQ3_S_DEV 21
#define PHX_IQ2_S_DEV 22
#define PHX_MAX_USED_DEV 16
#define PHX_MAX_EXPERTS_DEV 256

namespace phx {

// Kernel timing hook.  While a context profiles, every launch carries a start and a stop event that
// the runtime stamps with the kernel's own execution interval (hipExtLaunchKernel), the interval a
// kernel-trace profiler reports, so dispatch latency is not counted; inside a stream capture the two
// events become graph nodes around the launch; otherwise a plain launch.
struct LaunchTimer {
    virtual hipEvent_t event() = 0;
    virtual void done(hipEvent_t start, hipEvent_t stop) = 0;
    // inside a stream capture: the events become event-record nodes of the capture graph around a
    // plain launch (mark adds one after the stream's current capture dependencies)
    virtual bool capturing() const { return false; }
    virtual void mark(hipStream_t, hipEvent_t) {}
};
extern thread_local LaunchTimer* g_launch_timer;

// Fault injection for tests of the error paths: PHX_FAULT="malloc:n" or "launch:n", read when a context
// is created, fails that context's n-th device allocation with hipErrorOutOfMemory, or skips its n-th
// kernel launch and every later one of the same call and reports hipErrorLaunchFailure at the call's
// launch check (as a lost device would); one fault per context.
struct FaultPlan {
    enum Site { NONE = 0, MALLOC = 1, LAUNCH = 2 };
    int site = NONE;
    int64_t n = 0, count = 0;
    hipError_t pending = hipSuccess;
    bool fire(int s) { return site == s && n > 0 && ++count == n; }
};
extern thread_local FaultPlan* g_fault;  // the plan of the context whose call is running

template <typename... KArgs, typename... Args>
inline void launch(void (*kernel)(KArgs...), dim3 grid, dim3 block, uint32_t lds, hipStream_t st, Args... args)
{
    if (FaultPlan* f = g_fault) {
        if (f->pending != hipSuccess) return;  // after a fault nothing more runs in the call
        if (f->fire(FaultPlan::LAUNCH)) {
            f->pending = hipErrorLaunchFailure;
            return;
        }
    }
    if (LaunchTimer* t = g_launch_timer) {
        hipEvent_t a = t->event(), b = t->event();
        if (t->capturing()) {
            t->mark(st, a);
            hipLaunchKernelGGL(kernel, grid, block, lds, st, args...);
            t->mark(st, b);
        } else {
            hipExtLaunchKernelGGL(kernel, grid, block, lds, st, a, b, 0u, args...);
        }
        t->done(a, b);
    } else {
        hipLaunchKernelGGL(kernel, grid, block, lds, st, args...);
    }
}

constexpr int kRowGroup = 64;  // rows per interleaved row group: one wave64, lane = row

// Activation formats produced for each weight type.
enum ActFmt { ACT_Q8_0 = 0, ACT_K4 = 1, ACT_K6 = 2, ACT_Q8K = 3 };

// One stack of quantized matrices (experts, or one dense matrix), repacked at upload into row
// groups of 64 rows: payload[m][rg][b][lane][pay] and scale[m][rg][b][lane][sbytes], so the 64
// lanes of a wave read block b of 64 consecutive rows as one contiguous span.  A row group's payload
// is rg_pay bytes: for Q4_0 / Q8_0 its nb * 64 payload blocks are followed by the same fp16 scales
// grouped per lane by 8 blocks, [nb/8][lane][8] (one 16 B load gives a row the scales of 8
// consecutive blocks: the decode kernels' layout), so a row group's weights and scales share pages.
//   Q4_0: pay 16 (nibbles, low = element j, high = j+16), scale fp16 d
//   Q8_0: pay 32 (int8), scale fp16 d
//   Q4_K: pay 144 = 128 nibbles in (sub-block, l, m) order + sc[8] + m[8]; scale fp16 d | fp16 dmin << 16
//   Q6_K: pay 208 = 128 low-nibble plane + 64 high-bit plane + int8 sc[16]; scale fp16 d
//   IQ2_XXS / IQ2_S / IQ3_S: pay 64 / 80 / 112 = the block's bytes after d, unchanged (IQ3_S padded by 4);
//             scale fp16 d; grid points at the codebooks (iq_grids.h) expanded on the device
struct QMat {
    int type = -1;
    int n_mat = 0, rows = 0, cols = 0;  // cols includes any zero padding of K
    int rg = 0, nb = 0;                 // row groups, blocks (32 or 256 elements) per row
    int pay = 0, sbytes = 0;
    bool paired = false;                // gate|up: row group g = gate rows 32g..32g+31 and the matching up rows
    int64_t rg_pay = 0;                 // payload bytes per row group (blocks, then Q4_0 / Q8_0 scale groups)
    uint8_t* payload = nullptr;
    uint8_t* scale = nullptr;
    const void* grid = nullptr;         // IQ types: the context's expanded codebook of this type
    bool has_sc8() const { return type == PHX_Q4_0_DEV || type == PHX_Q8_0_DEV; }
    int64_t sc8_off() const { return (int64_t)nb * kRowGroup * pay; }  // scale groups within a row group
    int64_t mat_pay_stride() const { return (int64_t)rg * rg_pay; }
    int64_t mat_sc_stride() const { return (int64_t)rg * nb * kRowGroup * sbytes; }
};

// Quantized activation rows for one weight type.
//   ACT_Q8_0: q int8 [cols], d f32 [cols/32] (value of the fp16 scale), s int32 [cols/32] block sums
//   ACT_K4:   q int8 [cols] permuted per 32-sub-block as dwords (l, m) = x[32s + l + 8m],
//             d f32 [cols/256], s int32 [cols/16] (the Q8_K bsums)
//   ACT_K6:   q int32 [cols/256][8 P][8 l][2] masked pair dwords, d f32 [cols/256],
//             s int32 [cols/256][16 sub][8 l] offset terms -32*(x_l + x_{l+8})
//   ACT_Q8K:  q int8 [cols] in element order, d f32 [cols/256] (the IQ types' Q8_K input)
struct Act {
    int fmt = ACT_Q8_0;
    int cols = 0;
    int8_t* q = nullptr;
    int64_t qstride = 0;  // bytes per row
    float* d = nullptr;
    int dstride = 0;      // floats per row
    int* s = nullptr;
    int sstride = 0;      // ints per row
    uint16_t* qh = nullptr;  // optional: the same integers as fp16 bits [row][cols] (for MFMA); ACT_Q8_0 in
                             // element order, the K formats per super-block in the order [l][s][mm']:
                             // x(32 s + l + 8 {0, 2, 1, 3}[mm'])
    int64_t qhstride = 0;    // halves per row
    bool fold = false;       // ACT_Q8_0 with qh: qh holds fp16(q * d), the block scale folded in (the
                             // tolerance mode's operands), instead of the integers
    uint16_t* bh = nullptr;  // optional, K formats: the Q8_K block sums as fp16 [row][cols / 16]
    int64_t bhstride = 0;    // halves per row
};

struct Tile { int e, start, cnt; };
// decode-path tile: expert, assignment count (<= 2) and the assignment rows themselves
struct DecTile { int e, cnt, row[2]; };

// kernels.hip launchers (all enqueue on `st`)
void launch_prologue(hipStream_t st, int T, int d, float eps, const float* x, const float* gate_inp_scale,
                     const float* pre2, const float* ffn_norm, float* router_in, float* xscale, Act act_gu,
                     Act act_sh, int* flags);
// the router kernels' top-k outputs (ids set: ids [T][k] and weights, written by the router itself when one
// workgroup holds every expert, E <= 64; else ignored, k_topk runs)
struct TopkOut {
    int k = 0, rule = 0;
    const float* ds = nullptr;
    int* ids = nullptr;
    float* w = nullptr;
};
// xscale set: the router forms m from the layer input x (router_in = x), the prologue's row scales and the
// router input scale gis, where router_reads_x(T, d, E) (its many-token variant); otherwise router_in is m
struct RouterX {
    const float* xscale = nullptr;
    const float* gis = nullptr;
};
bool router_reads_x(int T, int d, int E);
void launch_router_exact(hipStream_t st, int T, int d, int E, const float* wt4, const float* router_in, float* logits,
                         TopkOut to = TopkOut{}, RouterX rx = RouterX{});
void launch_topk(hipStream_t st, int T, int E, int k, int rule, const float* logits, const float* down_scale,
                 int* ids, float* w);
void launch_dispatch(hipStream_t st, int n_assign, int E, int A, const int* ids, int* offsets, int* perm,
                     Tile* tiles, int* ntiles);
// req: the paired gate|up product's down input (gelu(g) * u as Q8_0 rows, req_rows of them), formed in
// the product's epilogue where it can be, else by k_requant after it
void launch_grouped(hipStream_t st, const QMat& w, Act act, const Tile* tiles, const int* ntiles, int max_tiles,
                    int A, const int* perm, int act_div, float* out0, float* out1, int split, int out_stride,
                    const Act* req = nullptr, const float* gelu_tab = nullptr, int req_rows = 0);
void launch_requant(hipStream_t st, int rows, int nf, const float* g, const float* u, const float* gelu_tab, Act act);
// standalone Q8_0 (fmt_k 0) / Q8_K (fmt_k 1) quantizer of rows x n inputs; mode as PHX_QUANT_*; -1 on a bad mode
int launch_quant(hipStream_t st, int fmt_k, int mode, int rows, int n, float eps, const float* x, const float* aux,
                 const float* tab, int8_t* qs, uint16_t* d16, float* dk, int16_t* bsums, int* flags);
// per row: x = (x + rmsnorm(y) * w) * s (s != 1), then with w2 the Q8_0 of rmsnorm(x) * w2 (n <= 16384)
void launch_norm_add(hipStream_t st, int rows, int n, float eps, float s, float* x, const float* y, const float* w,
                     const float* w2, int8_t* qs, uint16_t* d16, int* flags);
// dense Q4_0 / Q8_0 matvec of GGUF rows with planar Q8_0 input, T input rows; LDS bytes per launch
size_t matvec_lds(int type, int nb);
void launch_matvec(hipStream_t st, int type, int rows, int nb, int T, const uint8_t* w, const int8_t* xq,
                   const uint16_t* xd, float* y);
// prefill path (kernels_prefill.hip): Q4_0 / Q8_0 grouped products on MFMA, tiles of up to kMmaTile
// assignments; same arguments and outputs as launch_grouped.  npos > 0 reads the activations in
// expert-list order, block-major (fp16 integers of block b, list position p at qh + (b * npos + p) * 32,
// scales at d[b * npos + p]).  For a paired gate|up matrix with qout set, the kernel also does the
// GELU-gated requant into qout in that layout over qnpos positions (its qh and d only).  fold: the
// tolerance mode (scales folded into fp16 operands, the row accumulated on the matrix cores).
constexpr int kMmaTile = 128;
void launch_grouped_mfma(hipStream_t st, const QMat& w, Act act, const Tile* tiles, const int* ntiles, int max_tiles,
                         const int* perm, int act_div, float* out0, float* out1, int split, int out_stride,
                         int64_t npos = 0, const Act* qout = nullptr, int64_t qnpos = 0,
                         const float* gelu_tab = nullptr);
// K-quant prefill path (kernels_prefill.hip): Q4_K / Q6_K grouped products on MFMA, tiles of up to
// kKmmaTile assignments, activations' fp16 copies (qh; Q4_K also bh) in row order; arguments and outputs
// as launch_grouped
constexpr int kKmmaTile = 48;
void launch_grouped_kmma(hipStream_t st, const QMat& w, Act act, const Tile* tiles, const int* ntiles, int max_tiles,
                         const int* perm, int act_div, float* out0, float* out1, int split, int out_stride);
void launch_combine(hipStream_t st, int T, int d, int k, float eps, const float* yd, const float* w,
                    const float* shared, const float* post1, const float* post2, float* out, float* x_resid,
                    const float* post_ffw, int* flags);
void launch_combine_wide(hipStream_t st, int T, int d, int k, float eps, const float* yd, const float* w,
                    const float* shared, const float* post1, const float* post2, float* out, float* x_resid,
                    const float* post_ffw, int* flags);
// decode path (kernels_decode.hip): four launches per layer for T <= 16 tokens, Q4_0 / Q8_0
struct DecLayerH {
    int T, d, E, k, nf, nff, rule, max_tiles;
    int seq = 0;  // position in a captured stack (the instrumented build's clock-stamp slot)
    int ncu;  // compute units: the gate|up launch has at most one unit workgroup per CU
    float eps;
    const float *x, *W, *gis, *ds, *pre2, *post1, *post2, *fnorm, *post_ffw, *shared_in;
    const float* xscale = nullptr;  // [T] rms scales formed earlier in the call (the exact selection reuses them)
    const QMat *gu, *dn, *sgu, *sdn;  // sgu / sdn null: no shared FFN computed in the call
    double *Lb, *Bb;
    uint32_t* kb;  // [T][E][4] selection keys of the certified router (see k_dec_route)
    int* bad = nullptr;  // [1 + T] the count and the tokens the certified selection leaves to the exact chains
    int *ids, *offsets, *perm, *flags;
    float *w, *logits, *g, *u, *yd, *shg, *shu, *shout, *out, *xres;
    const float* xin = nullptr;  // the residual's source rows when not xres itself
    DecTile* tiles;
    Act agu, ash, adn, asd;  // packed Q8_0 rows: expert and shared inputs [T], down inputs [T*k], [T]
    const float* gelu_tab;
};
bool dec_supported(const DecLayerH& h);
void launch_dec_route(hipStream_t st, const DecLayerH& h);
// the general path's selection from k_dec_route's certified sums: ids, weights and logits per token
void launch_cert_select(hipStream_t st, const DecLayerH& h);
// whether launch_cert_select runs as one launch (a workgroup per token in at most two rounds over the
// compute units) rather than a wave per token and a fallback launch for the uncertified tokens
inline bool cert_select_one_launch(const DecLayerH& h) { return h.T <= 2 * std::max(h.ncu, 1); }
// the certified router for many tokens: matrix-core logits with bounds (Lb, Bb) and selection keys kb
// [T][E][4] for launch_cert_select, from x and the router rows prescaled at upload (Ws[e][i] =
// fl(s_i W[e][i]), s the router scale) with their squared norms over the kernel's kRouterRanges
// reduction ranges (Wn[e][r], rounded up); it forms the rows' rms scales itself (xscale out), so it
// needs nothing from the prologue
constexpr int kRouterRanges = 8;
// reduction range r of a row of d elements (d % 16 == 0): chunks of 16 elements [c0, c0 + cnt)
__host__ __device__ inline void router_range(int d, int r, int* c0, int* cnt)
{
    const int nch = d / 16, base = nch / kRouterRanges, extra = nch % kRouterRanges;
    *c0 = r * base + (r < extra ? r : extra);
    *cnt = base + (r < extra);
}
bool router_mm_supported(int T, int d, int E);
void launch_router_mm(hipStream_t st, int T, int d, int E, float eps, const float* x, const float* Ws, const float* Wn,
                      float* xscale, double* Lb, double* Bb, uint32_t* kb, int* cbad, int* flags);
// a stack layer's router with the previous layer's combine folded in (prev: that layer, its xin the
// rows it reads, its xres where the new x goes; h.x must be prev.xres)
void launch_dec_route_fused(hipStream_t st, const DecLayerH& prev, const DecLayerH& h);
void launch_dec_gu(hipStream_t st, const DecLayerH& h);
void launch_dec_down(hipStream_t st, const DecLayerH& h);
void launch_dec_combine(hipStream_t st, const DecLayerH& h);
void launch_stream_read(hipStream_t st, const void* src, int64_t bytes, uint32_t* sink);
void launch_stream_copy(hipStream_t st, void* dst, const void* src, int64_t bytes);
void launch_fill_u32(hipStream_t st, uint32_t* p, int64_t n, uint32_t v);
// a small copy (bytes a multiple of 16, either side may be pinned host memory) as one kernel
void launch_copy_small(hipStream_t st, void* dst, const void* src, int64_t bytes);
// the last copies of a host-buffer call (d1 / s1 may be null), then *done = ++*ctr (ctr device memory,
// done pinned host memory) after a system-scope fence; one workgroup
void launch_copy_done(hipStream_t st, void* d0, const void* s0, void* d1, const void* s1, int64_t bytes, uint32_t* ctr,
                      uint32_t* done);
void launch_planar_act(hipStream_t st, int rows, int n, const int8_t* qs, const uint16_t* d, Act a);
// planar Q8_K rows (qs [rows][n], d [rows][n/256]) into a's K-quant orders (ACT_K4 / ACT_K6, qh / bh when set)
void launch_planar_act_k(hipStream_t st, int rows, int n, const int8_t* qs, const float* d, Act a);
void launch_selftest(hipStream_t st, int op, int n, const float* a, const float* b, float* out, const float* gelu_tab);
void launch_selftest_seq(hipStream_t st, int m, int rows, const float* a, float* out);

}  // namespace phx
