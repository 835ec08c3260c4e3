// libphxmoe.so host runtime: the C ABI of include/phx_moe.h.  Owns the HIP device, one stream, all
// device memory, the per-layer repacked weights and the workspace; enqueues the kernels of
// kernels.hip for one MoE FFN block (the sequence GemmaGpu records at src/GemmaGpu.cs:683-704 and
// :850-882, with the CPU reference's arithmetic), and captures consecutive layers into a HIP graph.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <chrono>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "iq_grids.h"
#include "phx_internal.h"

using namespace phx;

namespace phx {
thread_local LaunchTimer* g_launch_timer = nullptr;
thread_local FaultPlan* g_fault = nullptr;
}

namespace {

// ------------------------------------------------------------------------------ host fp16 (RNE)
uint16_t half_bits(float value)
{
    uint32_t f;
    memcpy(&f, &value, 4);
    uint32_t sign = (f >> 16) & 0x8000u;
    int e = (int)((f >> 23) & 0xFF);
    uint32_t m = f & 0x7FFFFFu;
    if (e == 255) return (uint16_t)(sign | 0x7C00u | (m ? 0x200u : 0u));
    int ne = e - 112;
    if (ne >= 31) return (uint16_t)(sign | 0x7C00u);
    if (ne <= 0) {
        if (ne < -10) return (uint16_t)sign;
        m |= 0x800000u;
        int sh = 14 - ne;
        uint32_t hm = m >> sh, rem = m & ((1u << sh) - 1), half = 1u << (sh - 1);
        if (rem > half || (rem == half && (hm & 1))) hm++;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = sign | ((uint32_t)ne << 10) | (m >> 13), r = m & 0x1FFFu;
    if (r > 0x1000u || (r == 0x1000u && (h & 1))) h++;
    return (uint16_t)h;
}

float half_value(uint16_t h)
{
    uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1F, m = h & 0x3FF, bits;
    if (e == 0) {
        if (!m) bits = s;
        else {
            int k = -1;
            do { k++; m <<= 1; } while (!(m & 0x400));
            bits = s | (uint32_t)(112 - k) << 23 | (m & 0x3FF) << 13;
        }
    } else if (e == 31) bits = s | 0x7F800000u | m << 13;
    else bits = s | (e + 112) << 23 | m << 13;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

// GELU over the 65,536 fp16 inputs, the reference formula (src/CpuRefGemma.cs:85-92) evaluated in
// binary32 with a binary64 tanh: the table the kernels read for |x| < 10.
void build_gelu_table(std::vector<float>& tab)
{
    tab.resize(65536);
    for (int i = 0; i < 65536; i++) {
        float h = half_value((uint16_t)i);
        float g;
        if (!(h == h) || h <= -10.0f) g = 0.0f;
        else if (h >= 10.0f) g = h;
        else {
            float inner = 0.79788456080286535587989211986876f * h * (1.0f + 0.044715f * h * h);
            float v = 0.5f * h * (1.0f + (float)tanh((double)inner));
            g = half_value(half_bits(v));
        }
        tab[i] = g;
    }
}

int64_t row_bytes(int type, int cols)
{
    switch (type) {
    case PHX_F32: return (int64_t)cols * 4;
    case PHX_Q4_0: return (int64_t)(cols / 32) * 18;
    case PHX_Q8_0: return (int64_t)(cols / 32) * 34;
    case PHX_Q3_K: return (int64_t)(cols / 256) * 110;
    case PHX_Q4_K: return (int64_t)(cols / 256) * 144;
    case PHX_Q5_K: return (int64_t)(cols / 256) * 176;
    case PHX_Q6_K: return (int64_t)(cols / 256) * 210;
    case PHX_IQ2_XXS: return (int64_t)(cols / 256) * 66;
    case PHX_IQ2_S: return (int64_t)(cols / 256) * 82;
    case PHX_IQ3_S: return (int64_t)(cols / 256) * 110;
    }
    return -1;
}

bool iq_type(int t) { return t == PHX_IQ2_XXS || t == PHX_IQ2_S || t == PHX_IQ3_S; }
bool k_type(int t) { return t == PHX_Q3_K || t == PHX_Q4_K || t == PHX_Q5_K || t == PHX_Q6_K; }
bool quant_type(int t) { return t == PHX_Q4_0 || t == PHX_Q8_0 || k_type(t) || iq_type(t); }
int block_elems(int t) { return (t == PHX_Q4_0 || t == PHX_Q8_0) ? 32 : 256; }
// Q3_K rows live on the device as Q6_K blocks: DotK's integer lanes, float lanes and fold are the same
// for both (src/CpuRefKQuants.cs:183-211: sixteen scales of 16 elements, no min term), and every Q3_K
// value (q - 4 in -4..3, scale - 32 in -32..31, the same fp16 d) is a Q6_K one, so the Q6_K kernels give
// the reference's Q3_K results bit for bit
int dev_type(int t) { return t == PHX_Q3_K ? PHX_Q6_K : t; }
int act_fmt(int t)
{
    t = dev_type(t);
    return (t == PHX_Q4_K || t == PHX_Q5_K) ? ACT_K4 : t == PHX_Q6_K ? ACT_K6 : iq_type(t) ? ACT_Q8K : ACT_Q8_0;
}
int iq_pay(int t) { return t == PHX_IQ2_XXS ? 64 : t == PHX_IQ2_S ? 80 : 112; }
int round_up(int v, int m) { return (v + m - 1) / m * m; }

// ------------------------------------------------------------------------------ repack
// GGUF rows [n_mat][rows][row_bytes] -> row groups of 64 (see QMat).
struct HostQ {
    std::vector<uint8_t> payload, scale;
};

// the eight 6-bit scales and mins of a Q4_K / Q5_K block (ScaleMinK4, src/CpuRefKQuants.cs:32-43)
void decode_k4_scales(const uint8_t* blk, int* sc, int* mn)
{
    const uint8_t* s8 = blk + 4;
    for (int j = 0; j < 8; j++) {
        if (j < 4) { sc[j] = s8[j] & 63; mn[j] = s8[j + 4] & 63; }
        else { sc[j] = (s8[j + 4] & 0xF) | ((s8[j - 4] >> 6) << 4); mn[j] = (s8[j + 4] >> 4) | ((s8[j] >> 6) << 4); }
    }
}

void decode_q4k_natural(const uint8_t* blk, uint8_t* q, int* sc, int* mn)
{
    // UnpackK's element order for Q4_K (src/CpuRefKQuants.cs:118-133)
    decode_k4_scales(blk, sc, mn);
    const uint8_t* q4 = blk + 16;
    for (int c = 0; c < 4; c++)
        for (int l = 0; l < 32; l++) {
            q[64 * c + l] = q4[32 * c + l] & 0xF;
            q[64 * c + 32 + l] = q4[32 * c + l] >> 4;
        }
}

void decode_q5k_natural(const uint8_t* blk, uint8_t* q, int* sc, int* mn)
{
    // UnpackK's element order for Q5_K (src/CpuRefKQuants.cs:134-146): Q4_K's nibbles plus bit j of qh[l]
    // as the fifth bit of element l of sub-block j
    decode_k4_scales(blk, sc, mn);
    const uint8_t* qh = blk + 16;
    const uint8_t* q4 = blk + 48;
    for (int c = 0; c < 4; c++)
        for (int l = 0; l < 32; l++) {
            q[64 * c + l] = (uint8_t)((q4[32 * c + l] & 0xF) | (((qh[l] >> (2 * c)) & 1) << 4));
            q[64 * c + 32 + l] = (uint8_t)((q4[32 * c + l] >> 4) | (((qh[l] >> (2 * c + 1)) & 1) << 4));
        }
}

// One Q3_K block (110 B) as the Q6_K block (210 B) of the same values: q6 = q3 + 32, scale = scale - 32,
// d unchanged (UnpackQ3K, src/CpuRefIQuants.cs:28-43; ScaleQ3K :19-25)
void q3k_as_q6k(const uint8_t* blk, uint8_t* out)
{
    const uint8_t* hm = blk;
    const uint8_t* q3 = blk + 32;
    const uint8_t* s8 = blk + 96;
    uint8_t v[256];
    for (int h = 0; h < 2; h++)
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 32; l++) {
                const int a = ((q3[32 * h + l] >> (2 * j)) & 3) - ((hm[l] >> (4 * h + j)) & 1 ? 0 : 4);
                v[128 * h + 32 * j + l] = (uint8_t)(a + 32);
            }
    memset(out, 0, 210);
    for (int n = 0; n < 2; n++) {
        const uint8_t* a = v + 128 * n;
        uint8_t* L = out + 64 * n;
        uint8_t* H = out + 128 + 32 * n;
        for (int l = 0; l < 32; l++) {
            L[l] = (uint8_t)((a[l] & 0xF) | ((a[l + 64] & 0xF) << 4));
            L[l + 32] = (uint8_t)((a[l + 32] & 0xF) | ((a[l + 96] & 0xF) << 4));
            H[l] = (uint8_t)((a[l] >> 4) | ((a[l + 32] >> 4) << 2) | ((a[l + 64] >> 4) << 4) | ((a[l + 96] >> 4) << 6));
        }
    }
    for (int j = 0; j < 16; j++) {
        const int lo = j < 8 ? s8[j] & 0xF : s8[j - 8] >> 4;
        const int hi = (s8[8 + (j & 3)] >> (2 * (j >> 2))) & 3;
        out[192 + j] = (uint8_t)(int8_t)((lo | (hi << 4)) - 32);
    }
    out[208] = blk[108];
    out[209] = blk[109];
}

void decode_q6k_natural(const uint8_t* blk, uint8_t* v)
{
    // UnpackK's element order for Q6_K (src/CpuRefKQuants.cs:98-111), kept unsigned (q + 32)
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    for (int n = 0; n < 2; n++) {
        uint8_t* a = v + 128 * n;
        for (int l = 0; l < 32; l++) {
            a[l] = (uint8_t)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4));
            a[l + 32] = (uint8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4));
            a[l + 64] = (uint8_t)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4));
            a[l + 96] = (uint8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4));
        }
        ql += 64;
        qh += 32;
    }
}

void repack_block(int type, const uint8_t* blk, uint8_t* pay, uint8_t* sc)
{
    switch (type) {
    case PHX_Q4_0:
        memcpy(sc, blk, 2);
        memcpy(pay, blk + 2, 16);
        break;
    case PHX_Q8_0:
        memcpy(sc, blk, 2);
        memcpy(pay, blk + 2, 32);
        break;
    case PHX_Q4_K:
    case PHX_Q5_K: {
        // 128 nibble bytes: dword w = 2 value dwords (s, l = 2 (w % 4), +1), byte mm of each the element
        // 32 s + l + 8 mm; then 8 scales and 8 mins; Q5_K then 8 dwords of fifth bits: bit l of byte mm of
        // dword s is element 32 s + l + 8 mm's
        uint8_t q[256];
        int s[8], m[8];
        if (type == PHX_Q4_K) decode_q4k_natural(blk, q, s, m);
        else decode_q5k_natural(blk, q, s, m);
        for (int w = 0; w < 32; w++) {
            int sb = w / 4, p = w % 4;
            for (int mm = 0; mm < 4; mm++)
                pay[4 * w + mm] = (uint8_t)((q[32 * sb + 2 * p + 8 * mm] & 0xF) | ((q[32 * sb + 2 * p + 1 + 8 * mm] & 0xF) << 4));
        }
        for (int j = 0; j < 8; j++) { pay[128 + j] = (uint8_t)s[j]; pay[136 + j] = (uint8_t)m[j]; }
        if (type == PHX_Q5_K) {
            for (int sb = 0; sb < 8; sb++)
                for (int mm = 0; mm < 4; mm++) {
                    uint8_t b = 0;
                    for (int l = 0; l < 8; l++) b |= (uint8_t)(((q[32 * sb + l + 8 * mm] >> 4) & 1) << l);
                    pay[144 + 4 * sb + mm] = b;
                }
        }
        memcpy(sc, blk, 4);  // d | dmin << 16
        break;
    }
    case PHX_Q3_K: {
        uint8_t q6[210];
        q3k_as_q6k(blk, q6);
        repack_block(PHX_Q6_K, q6, pay, sc);
        break;
    }
    case PHX_Q6_K: {
        uint8_t v[256], out[256];
        decode_q6k_natural(blk, v);
        for (int P = 0; P < 8; P++)
            for (int l = 0; l < 8; l++) {
                uint8_t* o = out + 4 * (P * 8 + l);
                o[0] = v[32 * P + l];
                o[1] = v[32 * P + l + 8];
                o[2] = v[32 * P + 16 + l];
                o[3] = v[32 * P + 16 + l + 8];
            }
        for (int w = 0; w < 32; w++)
            for (int mm = 0; mm < 4; mm++)
                pay[4 * w + mm] = (uint8_t)((out[4 * (2 * w) + mm] & 0xF) | ((out[4 * (2 * w + 1) + mm] & 0xF) << 4));
        for (int h = 0; h < 16; h++)
            for (int mm = 0; mm < 4; mm++) {
                uint8_t b = 0;
                for (int i = 0; i < 4; i++) b |= (uint8_t)(((out[4 * (4 * h + i) + mm] >> 4) & 3) << (2 * i));
                pay[128 + 4 * h + mm] = b;
            }
        memcpy(pay + 192, blk + 192, 16);
        memcpy(sc, blk + 208, 2);
        break;
    }
    case PHX_IQ2_XXS:
    case PHX_IQ2_S:
    case PHX_IQ3_S:  // the bytes after d unchanged (IQ3_S's 108 padded to 112 by the zeroed buffer)
        memcpy(sc, blk, 2);
        memcpy(pay, blk + 2, (size_t)(row_bytes(type, 256) - 2));
        break;
    }
}

// paired: rows are [gate (rows/2) | up (rows/2)]; row group g holds gate rows 32g..32g+31 in lanes 0-31
// and up rows rows/2 + 32g.. in lanes 32-63.
void repack(int type, const uint8_t* src, int n_mat, int rows, int cols, QMat& q, HostQ& h, bool paired = false)
{
    q.type = dev_type(type);
    q.n_mat = n_mat;
    q.rows = rows;
    q.cols = cols;
    q.paired = paired;
    q.rg = paired ? (rows / 2 + 31) / 32 : (rows + kRowGroup - 1) / kRowGroup;
    q.nb = cols / block_elems(type);
    q.pay = type == PHX_Q4_0 ? 16 : type == PHX_Q8_0 ? 32 : type == PHX_Q4_K ? 144 : type == PHX_Q5_K ? 176
          : iq_type(type) ? iq_pay(type) : 208;
    q.sbytes = (type == PHX_Q4_K || type == PHX_Q5_K) ? 4 : 2;
    const int64_t rb = row_bytes(type, cols), bb = rb / q.nb;
    const int nb8 = (q.nb + 7) / 8;
    q.rg_pay = (int64_t)q.nb * kRowGroup * q.pay + (q.has_sc8() ? (int64_t)nb8 * kRowGroup * 16 : 0);
    h.payload.assign((size_t)q.mat_pay_stride() * n_mat, 0);
    h.scale.assign((size_t)q.mat_sc_stride() * n_mat, 0);
    const int64_t total_rows = (int64_t)n_mat * rows;
    unsigned nt = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
    std::vector<std::thread> th;
    for (unsigned w = 0; w < nt; w++) {
        th.emplace_back([&, w]() {
            for (int64_t gr = w; gr < total_rows; gr += nt) {
                int m = (int)(gr / rows), r = (int)(gr % rows);
                int rg = r / kRowGroup, lane = r % kRowGroup;
                if (paired) {
                    const int half = rows / 2, up = r >= half, j = up ? r - half : r;
                    rg = j / 32;
                    lane = (j % 32) + (up ? 32 : 0);
                }
                const uint8_t* row = src + gr * rb;
                uint8_t* rgp = h.payload.data() + ((int64_t)m * q.rg + rg) * q.rg_pay;
                for (int b = 0; b < q.nb; b++) {
                    int64_t idx = (((int64_t)m * q.rg + rg) * q.nb + b) * kRowGroup + lane;
                    repack_block(type, row + b * bb, rgp + ((int64_t)b * kRowGroup + lane) * q.pay,
                                 h.scale.data() + idx * q.sbytes);
                }
            }
        });
    }
    for (auto& t : th) t.join();
    if (q.has_sc8()) {
        // each row group's scale groups [b / 8][lane][8] fp16 after its payload blocks
        const uint16_t* s1 = (const uint16_t*)h.scale.data();
        for (int64_t mr = 0; mr < (int64_t)n_mat * q.rg; mr++) {
            uint16_t* s8 = (uint16_t*)(h.payload.data() + mr * q.rg_pay + q.sc8_off());
            for (int b = 0; b < q.nb; b++)
                for (int lane = 0; lane < kRowGroup; lane++)
                    s8[((b / 8) * kRowGroup + lane) * 8 + b % 8] = s1[(mr * q.nb + b) * kRowGroup + lane];
        }
    }
}

struct Layer {
    bool present = false;
    phx_moe_layer_desc desc{};
    float *wt4 = nullptr, *wrow = nullptr, *gis = nullptr, *ds = nullptr, *pre2 = nullptr, *post1 = nullptr, *post2 = nullptr;
    float *wsc = nullptr, *wnr = nullptr;  // the many-token router's prescaled rows and their range norms^2
    float *ffn_norm = nullptr, *post_ffw = nullptr;
    QMat gu, dn, sgu, sdn;
    uint64_t gen = 0;  // upload generation: graphs captured over an earlier upload are stale
};

struct Buf {
    void* p = nullptr;
    size_t bytes = 0;
};

}  // namespace

struct phx_moe_ctx {
    int device = 0;
    int ncu = 256;  // compute units of the device
    hipStream_t stream = nullptr;
    // the general path's prologue runs on side beside the matrix-core router (fork and join events)
    hipStream_t side = nullptr;
    hipEvent_t ev_fork = nullptr, ev_join = nullptr;
    std::string err;
    float* gelu_tab = nullptr;
    std::vector<Layer> layers;
    std::vector<Buf> ws;
    int* flags = nullptr;  // [0] count of certified-sum fallbacks, [1] router fallbacks, [15] host-call completions
    int last_T = 0, last_layer = -1;
    // profiling
    bool profiling = false;
    struct Pending { int kind; hipEvent_t a, b; bool first = true; };  // first: the call's first kernel
    std::vector<Pending> pending;
    std::vector<Pending> graph_timing;  // event pairs recorded inside the captured stack
    bool capturing = false;
    std::vector<hipEvent_t> pool;
    double prof_ms[PHX_K_COUNT] = {};
    int64_t prof_calls[PHX_K_COUNT] = {};
    // stack graph
    hipGraphExec_t graph_exec = nullptr;
    hipGraph_t graph = nullptr;
    int graph_T = 0, graph_first = 0, graph_n = 0;
    bool graph_gu_kept = true;  // the captured stack's last layer stores g and u
    // what the stack graph was captured over: each layer's upload generation and the workspace
    // pointers (a later upload or a workspace regrowth frees memory the graph still names)
    std::vector<uint64_t> graph_gens;
    std::vector<void*> graph_ws;
    int64_t ffn_graph_hits = 0, ffn_graph_misses = 0;  // host-buffer call graphs (ffn_host)
    // phx_moe_ffn_noalloc: this device's address of the scratch array, the workspace table laid out
    // inside it (sized at creation, swapped with ws during a call), whether the last call used it, and
    // the bump allocation ensure() does while it lays the table out
    unsigned char* scratch = nullptr;
    std::vector<Buf> ws_scratch;
    // the IQ codebooks expanded (iq_grids.h): IQ2_XXS 256 and IQ2_S 1024 64-bit words, IQ3_S 512 32-bit
    uint8_t* iq_grid = nullptr;
    bool last_scratch = false;
    bool last_gu_kept = true;  // the last call stored the gate and up products (see keeps_gu)
    unsigned char* bump_base = nullptr;
    size_t bump_off = 0, bump_cap = 0;
    FaultPlan fault;  // PHX_FAULT, see phx_internal.h
    // phx_moe_ffn on host buffers: pinned staging rows ([3][pin_bytes]: x, shared, out) and each
    // (layer, T, flags, shared given) call captured once as a graph over the workspace it was captured on
    float* pin = nullptr;    // ... then the completion word (small calls)
    size_t pin_bytes = 0;
    struct FfnGraph {
        int layer, T;
        unsigned key;
        uint64_t gen;
        std::vector<void*> ws;
        hipGraphExec_t exec;
    };
    std::vector<FfnGraph> ffn_graphs;
    uint64_t upload_gen = 0;
};

namespace {

int set_err(phx_moe_ctx* c, int code, const char* fmt, ...)
{
    if (c) {
        char buf[512];
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(buf, sizeof buf, fmt, ap);
        va_end(ap);
        c->err = buf;
    }
    return code;
}

int hip_code(hipError_t e)
{
    switch (e) {
    case hipSuccess: return PHX_OK;
    case hipErrorOutOfMemory: return PHX_ERR_OOM;
    case hipErrorIllegalAddress:
    case hipErrorLaunchFailure:
    case hipErrorNoDevice: return PHX_ERR_DEVICE_LOST;
    default: return PHX_ERR_HIP;
    }
}

#define HIPCHK(c, expr)                                                                                       \
    do {                                                                                                      \
        hipError_t e_ = (expr);                                                                               \
        if (e_ != hipSuccess) return set_err(c, hip_code(e_), "%s: %s", #expr, hipGetErrorString(e_));        \
    } while (0)

// every device allocation of a context (the fault plan may fail it)
hipError_t dev_malloc(phx_moe_ctx* c, void** p, size_t n)
{
    if (c && c->fault.fire(FaultPlan::MALLOC)) {
        *p = nullptr;
        return hipErrorOutOfMemory;
    }
    return hipMalloc(p, n);  // the one device allocation site
}

// pinned host memory, under the same fault plan
hipError_t host_malloc(phx_moe_ctx* c, void** p, size_t n)
{
    if (c && c->fault.fire(FaultPlan::MALLOC)) {
        *p = nullptr;
        return hipErrorOutOfMemory;
    }
    return hipHostMalloc(p, n, hipHostMallocCoherent);
}

void drop_ffn_graphs(phx_moe_ctx* c)
{
    for (auto& g : c->ffn_graphs) (void)hipGraphExecDestroy(g.exec);
    c->ffn_graphs.clear();
}

// the launches' status: an injected launch fault, else the runtime's last error
hipError_t launch_status(phx_moe_ctx* c)
{
    if (c && c->fault.pending != hipSuccess) {
        const hipError_t e = c->fault.pending;
        c->fault.pending = hipSuccess;
        (void)hipGetLastError();
        return e;
    }
    return hipGetLastError();
}

// an API call on context c: its device current and its fault plan visible to the launches
struct CtxScope {
    FaultPlan* prev;
    explicit CtxScope(phx_moe_ctx* c) : prev(g_fault)
    {
        c->fault.pending = hipSuccess;  // a fault is reported by the call it happened in
        g_fault = &c->fault;
    }
    ~CtxScope() { g_fault = prev; }
};
#define ENTER(c)               \
    CtxScope ctx_scope_(c);    \
    HIPCHK(c, hipSetDevice((c)->device))

enum WsId {
    W_X, W_SHARED, W_OUT, W_RIN, W_XSCALE, W_AGU_Q, W_AGU_D, W_AGU_S, W_ASH_Q, W_ASH_D, W_ASH_S, W_LOGITS, W_IDS, W_W,
    W_OFF, W_PERM, W_TILES, W_NTILES, W_G, W_U, W_ADN_Q, W_ADN_D, W_ADN_S, W_YD, W_SHG, W_SHU, W_ASD_Q, W_ASD_D,
    W_ASD_S, W_SHOUT, W_ZERO, W_STILES, W_SNTILES, W_SOFF, W_SPERM, W_LB, W_BB, W_ADEC, W_SDEC, W_AGUP, W_ASHP, W_AGU_H, W_ADN_H, W_ASH_H, W_ASD_H, W_X2,
    W_MM_IDS, W_MM_OFF, W_MM_PERM, W_MM_TILES, W_MM_NT, W_MM_D, W_MM_S, W_MM_H, W_AGU_BH, W_ADN_BH, W_MK_Q, W_MK_BH, W_KB,
    W_CBAD, W_RSCALE, W_COUNT
};

int ensure(phx_moe_ctx* c, int id, size_t bytes)
{
    if ((int)c->ws.size() < W_COUNT) c->ws.resize(W_COUNT);
    Buf& b = c->ws[id];
    if (b.bytes >= bytes && b.p) return PHX_OK;
    if (c->bump_base) {  // laying out phx_moe_ffn_noalloc's table inside the scratch array
        const size_t off = (c->bump_off + 255) & ~(size_t)255, n = std::max<size_t>(bytes, 256);
        if (off + n > c->bump_cap)
            return set_err(c, PHX_ERR_ARG, "the call's workspace exceeds the %zu-byte scratch array", c->bump_cap);
        b.p = c->bump_base + off;
        b.bytes = n;
        c->bump_off = off + n;
        return PHX_OK;
    }
    if (b.p) HIPCHK(c, hipFree(b.p));
    b.p = nullptr;
    b.bytes = 0;
    size_t n = std::max<size_t>(bytes, 256);
    HIPCHK(c, dev_malloc(c, &b.p, n));
    b.bytes = n;
    if (id == W_ZERO) HIPCHK(c, hipMemset(b.p, 0, n));
    return PHX_OK;
}

template <class T> T* wp(phx_moe_ctx* c, int id) { return (T*)c->ws[id].p; }

// sizes of an activation buffer of `rows` rows of `cols` elements in format fmt
void act_sizes(int fmt, int64_t rows, int cols, size_t& qb, size_t& db, size_t& sb)
{
    if (fmt == ACT_Q8_0) { qb = rows * cols; db = rows * (cols / 32) * 4; sb = rows * (cols / 32) * 4; }
    else if (fmt == ACT_K4) { qb = rows * cols; db = rows * (cols / 256) * 4; sb = rows * (cols / 16) * 4; }
    else if (fmt == ACT_Q8K) { qb = rows * cols; db = rows * (cols / 256) * 4; sb = 4; }
    else { qb = rows * (cols / 256) * 512; db = rows * (cols / 256) * 4; sb = rows * (cols / 256) * 128 * 4; }
}

Act make_act(phx_moe_ctx* c, int fmt, int cols, int qid, int did, int sid)
{
    Act a;
    a.fmt = fmt;
    a.cols = cols;
    a.q = wp<int8_t>(c, qid);
    a.d = wp<float>(c, did);
    a.s = wp<int>(c, sid);
    if (fmt == ACT_Q8_0) { a.qstride = cols; a.dstride = cols / 32; a.sstride = cols / 32; }
    else if (fmt == ACT_K4) { a.qstride = cols; a.dstride = cols / 256; a.sstride = cols / 16; }
    else if (fmt == ACT_Q8K) { a.qstride = cols; a.dstride = cols / 256; a.sstride = 0; }
    else { a.qstride = (int64_t)(cols / 256) * 512; a.dstride = cols / 256; a.sstride = (cols / 256) * 128; }
    return a;
}

// Q8_0 rows packed one row after another, each row q (cols bytes), d (cols/32 floats), s (cols/32
// ints) contiguous: the decode kernels copy a row with one run of dword loads.
Act make_act_packed(phx_moe_ctx* c, int cols, int id)
{
    Act a;
    a.fmt = ACT_Q8_0;
    a.cols = cols;
    const int nb = cols / 32;
    uint8_t* base = wp<uint8_t>(c, id);
    a.q = (int8_t*)base;
    a.qstride = (int64_t)nb * 40;
    a.d = (float*)(base + cols);
    a.dstride = nb * 10;
    a.s = (int*)(base + cols + nb * 4);
    a.sstride = nb * 10;
    return a;
}

int ensure_act(phx_moe_ctx* c, int fmt, int64_t rows, int cols, int qid, int did, int sid)
{
    size_t qb, db, sb;
    act_sizes(fmt, rows, cols, qb, db, sb);
    int rc;
    if ((rc = ensure(c, qid, qb)) || (rc = ensure(c, did, db)) || (rc = ensure(c, sid, sb))) return rc;
    return PHX_OK;
}

constexpr int kTileA = 4;  // assignments per grouped tile

bool mfma_type(int t);
// the K-quant matrix-core kernel takes Q4_K and Q6_K device rows (so Q3_K too); Q5_K runs the VALU rows
bool kmma_type(int t) { return dev_type(t) == PHX_Q4_K || dev_type(t) == PHX_Q6_K; }

int ensure_workspace(phx_moe_ctx* c, const Layer& L, int T)
{
    const phx_moe_layer_desc& D = L.desc;
    const int64_t n = (int64_t)T * D.n_used;
    int rc;
#define ENS(id, bytes) \
    if ((rc = ensure(c, id, (size_t)(bytes)))) return rc
    ENS(W_X, (size_t)T * D.d * 4);
    ENS(W_X2, (size_t)T * D.d * 4);  // a stack's second x row set (layers alternate between the two)
    ENS(W_SHARED, (size_t)T * D.d * 4);
    ENS(W_OUT, (size_t)T * D.d * 4);
    ENS(W_RIN, (size_t)T * D.d * 4);
    ENS(W_XSCALE, (size_t)T * 4);
    ENS(W_LOGITS, (size_t)T * D.n_expert * 4);
    ENS(W_IDS, n * 4);
    ENS(W_W, n * 4);
    ENS(W_OFF, (size_t)(D.n_expert + 1) * 4);
    ENS(W_PERM, n * 4);
    ENS(W_TILES, (size_t)((n + kTileA - 1) / kTileA + D.n_expert) * sizeof(Tile));
    ENS(W_NTILES, 4);
    ENS(W_G, n * D.n_ff * 4);
    ENS(W_LB, (size_t)T * D.n_expert * 8);
    ENS(W_BB, (size_t)T * D.n_expert * 8);
    ENS(W_KB, (size_t)T * D.n_expert * 16);
    ENS(W_CBAD, (size_t)(T + 1) * 4);
    ENS(W_RSCALE, (size_t)T * 4);
    ENS(W_U, n * D.n_ff * 4);
    ENS(W_YD, n * D.d * 4);
    if ((rc = ensure_act(c, act_fmt(D.gate_up_type), T, D.d, W_AGU_Q, W_AGU_D, W_AGU_S))) return rc;
    if ((rc = ensure_act(c, act_fmt(D.down_type), n, D.down_cols, W_ADN_Q, W_ADN_D, W_ADN_S))) return rc;
    if ((mfma_type(D.gate_up_type) && mfma_type(D.down_type)) || (kmma_type(D.gate_up_type) && kmma_type(D.down_type))) {
        // the matrix-core paths' fp16 activation copies (and the K path's fp16 block sums)
        ENS(W_AGU_H, (size_t)T * D.d * 2);
        ENS(W_ADN_H, (size_t)n * D.down_cols * 2);
        if (kmma_type(D.gate_up_type)) {
            ENS(W_AGU_BH, (size_t)T * (D.d / 16) * 2);
            ENS(W_ADN_BH, (size_t)n * (D.down_cols / 16) * 2);
        }
    }
    if (D.n_ff_shared > 0) {
        int scols = round_up(D.n_ff_shared, block_elems(D.shared_type));
        if ((rc = ensure_act(c, act_fmt(D.shared_type), T, D.d, W_ASH_Q, W_ASH_D, W_ASH_S))) return rc;
        if ((rc = ensure_act(c, act_fmt(D.shared_type), T, scols, W_ASD_Q, W_ASD_D, W_ASD_S))) return rc;
        if (mfma_type(D.shared_type)) {
            ENS(W_ASH_H, (size_t)T * D.d * 2);
            ENS(W_ASD_H, (size_t)T * scols * 2);
        }
        ENS(W_SHG, (size_t)T * D.n_ff_shared * 4);
        ENS(W_SHU, (size_t)T * D.n_ff_shared * 4);
        ENS(W_SHOUT, (size_t)T * D.d * 4);
        ENS(W_ZERO, (size_t)T * 4);
        ENS(W_STILES, (size_t)((T + kTileA - 1) / kTileA + 1) * sizeof(Tile));
        ENS(W_SNTILES, 4);
        ENS(W_SOFF, 8);
        ENS(W_SPERM, (size_t)T * 4);
    }
    ENS(W_TILES, (size_t)((n + 1) / 2 + D.n_expert) * sizeof(DecTile));
    ENS(W_ADEC, (size_t)n * (D.down_cols / 32) * 40);
    ENS(W_AGUP, (size_t)T * (D.d / 32) * 40);
    if (D.n_ff_shared > 0) ENS(W_ASHP, (size_t)T * (D.d / 32) * 40);
    if (D.n_ff_shared > 0) ENS(W_SDEC, (size_t)T * (D.n_ff_shared / 32) * 40);
#undef ENS
    return PHX_OK;
}

hipEvent_t get_event(phx_moe_ctx* c)
{
    if (!c->pool.empty()) {
        hipEvent_t e = c->pool.back();
        c->pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    (void)hipEventCreate(&e);
    return e;
}

// While profiling, the kernels launched inside a scope are timed one by one (their own execution
// intervals, see LaunchTimer); a kind's time per call is the sum over its kernels.
struct ProfScope : LaunchTimer {
    phx_moe_ctx* c;
    int kind;
    LaunchTimer* prev = nullptr;
    bool on = false, any = false;
    ProfScope(phx_moe_ctx* c_, int k) : c(c_), kind(k)
    {
        if (c->profiling) {
            on = true;
            if (!c->capturing) c->prof_calls[kind] += 1;
            prev = g_launch_timer;
            g_launch_timer = this;
        }
    }
    hipEvent_t event() override
    {
        if (!c->capturing) return get_event(c);
        hipEvent_t e = nullptr;  // owned by the captured graph's timing list
        (void)hipEventCreate(&e);
        return e;
    }
    void done(hipEvent_t a, hipEvent_t b) override
    {
        (c->capturing ? c->graph_timing : c->pending).push_back({kind, a, b, !any});
        any = true;
    }
    bool capturing() const override { return c->capturing; }
    // an event-record node after the capture's current dependencies, which then move past it (events
    // recorded through hipEventRecord inside a capture cannot be timed on this runtime)
    void mark(hipStream_t st, hipEvent_t e) override
    {
        hipStreamCaptureStatus status;
        unsigned long long id;
        hipGraph_t g;
        const hipGraphNode_t* deps;
        size_t nd;
        if (hipStreamGetCaptureInfo_v2(st, &status, &id, &g, &deps, &nd) != hipSuccess ||
            status != hipStreamCaptureStatusActive)
            return;
        hipGraphNode_t n;
        if (hipGraphAddEventRecordNode(&n, g, deps, nd, e) != hipSuccess) return;
        (void)hipStreamUpdateCaptureDependencies(st, &n, 1, hipStreamSetCaptureDependencies);
    }
    ~ProfScope()
    {
        if (on) g_launch_timer = prev;
    }
};

bool dec_type(int t) { return t == PHX_Q4_0 || t == PHX_Q8_0; }
bool mfma_type(int t) { return t == PHX_Q4_0 || t == PHX_Q8_0; }

// The decode path (kernels_decode.hip): few tokens, Q4_0/Q8_0 weights, K <= 4096.
DecLayerH dec_layer(phx_moe_ctx* c, const Layer& L, int T, const float* x, const float* shared, float* out, float* xres)
{
    const phx_moe_layer_desc& D = L.desc;
    const int n = T * D.n_used;
    const bool shared_ffn = shared == nullptr && D.n_ff_shared > 0;
    DecLayerH h{};
    h.T = T;
    h.d = D.d;
    h.E = D.n_expert;
    h.k = D.n_used;
    h.nf = D.n_ff;
    h.nff = D.n_ff_shared;
    h.rule = D.weight_rule;
    h.max_tiles = std::min(n, (n + 1) / 2 + D.n_expert);  // every tile holds one or two assignments
    h.ncu = c->ncu;
    h.eps = D.eps;
    h.x = x;
    h.W = L.wrow;
    h.gis = L.gis;
    h.ds = L.ds;
    h.pre2 = L.pre2;
    h.post1 = L.post1;
    h.post2 = L.post2;
    h.fnorm = L.ffn_norm;
    h.post_ffw = L.post_ffw;
    h.shared_in = shared;
    h.gu = &L.gu;
    h.dn = &L.dn;
    h.sgu = shared_ffn ? &L.sgu : nullptr;
    h.sdn = shared_ffn ? &L.sdn : nullptr;
    h.out = out;
    h.xres = xres;
    h.gelu_tab = c->gelu_tab;
    h.flags = c->flags;
    if (c->ws.size() >= (size_t)W_COUNT && c->ws[W_LB].p) {
        h.Lb = wp<double>(c, W_LB);
        h.Bb = wp<double>(c, W_BB);
        h.kb = wp<uint32_t>(c, W_KB);
        h.bad = wp<int>(c, W_CBAD);
        h.ids = wp<int>(c, W_IDS);
        h.offsets = wp<int>(c, W_OFF);
        h.perm = wp<int>(c, W_PERM);
        h.w = wp<float>(c, W_W);
        h.logits = wp<float>(c, W_LOGITS);
        h.g = wp<float>(c, W_G);
        h.u = wp<float>(c, W_U);
        h.yd = wp<float>(c, W_YD);
        h.tiles = wp<DecTile>(c, W_TILES);
        h.adn = make_act_packed(c, D.down_cols, W_ADEC);
        h.agu = make_act_packed(c, D.d, W_AGUP);
        if (shared_ffn) {
            h.shg = wp<float>(c, W_SHG);
            h.shu = wp<float>(c, W_SHU);
            h.shout = wp<float>(c, W_SHOUT);
            h.asd = make_act_packed(c, D.n_ff_shared, W_SDEC);
            h.ash = make_act_packed(c, D.d, W_ASHP);
        }
    }
    return h;
}

bool use_decode(phx_moe_ctx* c, const Layer& L, int T, unsigned flags)
{
    const phx_moe_layer_desc& D = L.desc;
    if (flags & PHX_FLAG_EXACT_ROUTER) return false;
    if (T > 16 || T * D.n_used > 256 || T * D.n_expert > 2048 || D.d > 4096 || D.d % 256 != 0) return false;
    if (!dec_type(D.gate_up_type) || D.down_type != D.gate_up_type) return false;
    if (D.n_ff_shared > 0 && D.shared_type != D.gate_up_type) return false;
    return dec_supported(dec_layer(c, L, T, nullptr, nullptr, nullptr, nullptr));
}

int run_layer_decode(phx_moe_ctx* c, const Layer& L, int T, const float* x, const float* shared, float* out, float* xres)
{
    hipStream_t st = c->stream;
    const DecLayerH h = dec_layer(c, L, T, x, shared, out, xres);
    {
        ProfScope p(c, PHX_K_ROUTER);
        launch_dec_route(st, h);
    }
    {
        ProfScope p(c, PHX_K_GATE_UP);
        launch_dec_gu(st, h);
    }
    {
        ProfScope p(c, PHX_K_DOWN);
        launch_dec_down(st, h);
    }
    {
        ProfScope p(c, PHX_K_COMBINE);
        launch_dec_combine(st, h);
    }
    HIPCHK(c, launch_status(c));
    return PHX_OK;
}

// Enqueue one MoE FFN block on the context stream (any T; exact router chains).
// The general path routes through the certified router (k_dec_route's double sums and bounds, then
// k_cert_select: the decode path's selection, exact chains for a token it cannot certify) where the
// router launch has few enough workgroups (T * E of them, each reading a router row) and the expert
// input is Q8_0 (k_dec_route writes it, with the matrix cores' fp16 copy where the rows carry one);
// otherwise, and always under PHX_FLAG_EXACT_ROUTER, through the exact float chains.
// The router workgroups also quantize the expert (and shared) input: workgroup (t, e) takes blocks
// e + g E for each of its eight-thread groups g, so the groups of a token's E workgroups must cover its
// d / 32 blocks.  With T * E > 1024 a workgroup has 256 threads (32 groups): d / 32 <= 32 E.
constexpr int CERT_MAX_TE = 8192;
bool cert_route(const Layer& L, int T, bool shared_ffn)
{
    const phx_moe_layer_desc& D = L.desc;
    if ((int64_t)T * D.n_expert > CERT_MAX_TE || D.d > 4096 || D.d % 256 != 0 || D.n_expert > 256) return false;
    if (D.d / 32 > 32 * D.n_expert) return false;
    if (!dec_type(D.gate_up_type) || (shared_ffn && !dec_type(D.shared_type))) return false;
    return true;
}

// prefill-sized expert work (several assignments per expert on average) runs on the matrix cores, whose
// kernels read the activations' fp16 copies
static bool mma_path(const phx_moe_layer_desc& D, int T)
{
    return mfma_type(D.gate_up_type) && mfma_type(D.down_type) && T * D.n_used >= 8 * D.n_expert;
}

// whether a call stores the gate and up products for phx_moe_get_intermediates: the matrix-core Q4_0 /
// Q8_0 products requantize gelu(g) * u in registers and store g and u only when asked to
bool keeps_gu(phx_moe_ctx* c, const Layer& L, int T, unsigned flags)
{
    return (flags & PHX_FLAG_KEEP_INTERMEDIATES) || use_decode(c, L, T, flags) || !mma_path(L.desc, T);
}

int run_layer_general(phx_moe_ctx* c, const Layer& L, int T, const float* x, const float* shared, float* out, float* xres,
                      bool exact, bool fast, bool keep)
{
    const phx_moe_layer_desc& D = L.desc;
    hipStream_t st = c->stream;
    const int d = D.d, E = D.n_expert, k = D.n_used, nf = D.n_ff;
    const int n = T * k;
    const bool shared_ffn = shared == nullptr && D.n_ff_shared > 0;
    const bool mma = mma_path(D, T);
    const bool kmma = kmma_type(D.gate_up_type) && kmma_type(D.down_type) && n >= 8 * E;
    const bool smma = shared_ffn && mfma_type(D.shared_type) && T >= 32;
    Act agu = make_act(c, act_fmt(D.gate_up_type), d, W_AGU_Q, W_AGU_D, W_AGU_S);
    if (mma || kmma) {
        agu.qh = wp<uint16_t>(c, W_AGU_H);
        agu.qhstride = d;
    }
    // the tolerance mode (the matrix-core products): every fp16 activation copy carries its block scale
    // folded in, which selects the tolerance-mode products
    agu.fold = fast && (mma || kmma);
    if (kmma && D.gate_up_type == PHX_Q4_K) {
        agu.bh = wp<uint16_t>(c, W_AGU_BH);
        agu.bhstride = d / 16;
    }
    Act ash;
    if (shared_ffn) ash = make_act(c, act_fmt(D.shared_type), d, W_ASH_Q, W_ASH_D, W_ASH_S);
    ash.cols = shared_ffn ? ash.cols : 0;
    if (smma) {
        ash.qh = wp<uint16_t>(c, W_ASH_H);
        ash.qhstride = d;
        ash.fold = fast;
    }
    // the certified routers (decode-style workgroups per pair up to CERT_MAX_TE pairs, the matrix-core
    // one beyond), else the exact chains
    const bool cert = !exact && cert_route(L, T, shared_ffn);
    const bool mmr = !exact && !cert && (int64_t)T * E > CERT_MAX_TE && router_mm_supported(T, d, E);
    bool joined = false;  // the side stream's prologue still to be joined
    if (cert) {
        // the router's certified sums with the expert (and shared) inputs quantized beside them, then
        // the selection
        DecLayerH h = dec_layer(c, L, T, x, shared, out, xres);
        h.agu = agu;
        h.ash = ash;
        {
            ProfScope p(c, PHX_K_ROUTER);
            launch_dec_route(st, h);
        }
        {
            ProfScope p(c, PHX_K_TOPK);
            launch_cert_select(st, h);
        }
    } else {
        // the many-token routers form their input m from x and the row scales themselves (no m rows written)
        const bool rx = mmr || router_reads_x(T, d, E);
        // the matrix-core products read only the fp16 copies of their inputs: no int8 rows or sums
        Act pgu = agu, psh = ash;
        if (mma || kmma) pgu.q = nullptr, pgu.s = nullptr;
        if (smma) psh.q = nullptr, psh.s = nullptr;
        // the matrix-core router needs nothing from the prologue: the prologue runs on the side stream
        // (launched after the router, whose workgroups need more LDS than a prologue-filled compute unit
        // leaves), joined before the products read its rows.  Beside a one-launch selection it starts
        // once the router is done: the router alone is faster (C4 18.6 -> 16.1 us) and the prologue
        // takes the compute units the selection's rounds leave (layer 0.493 -> 0.485 ms).  Beside the
        // two-kernel selection it starts with the router: after it, it slowed the fallback's exact
        // chains more than it sped the router (C3 router 31.4 -> 26.8 us, selection 24.8 -> 32.1 us).
        auto prologue = [&](hipStream_t sp) {
            ProfScope p(c, PHX_K_PROLOGUE);
            launch_prologue(sp, T, d, D.eps, x, L.gis, L.pre2, shared_ffn ? L.ffn_norm : nullptr,
                            rx ? nullptr : wp<float>(c, W_RIN), wp<float>(c, W_XSCALE), pgu, psh, c->flags);
        };
        if (!mmr) prologue(st);
        // up to 64 experts the router's waves hold all of a token's logits and take its top-k themselves
        const bool fused_topk = E <= 64;
        if (mmr) {
            // matrix-core sums with bounds, then the certified selection (exact chains for the tokens
            // whose order the bounds leave open)
            DecLayerH h = dec_layer(c, L, T, x, shared, out, xres);
            h.xscale = wp<float>(c, W_RSCALE);
            const bool late = cert_select_one_launch(h);
            if (!late) HIPCHK(c, hipEventRecord(c->ev_fork, st));
            {
                ProfScope p(c, PHX_K_ROUTER);
                launch_router_mm(st, T, d, E, D.eps, x, L.wsc, L.wnr, wp<float>(c, W_RSCALE), h.Lb, h.Bb, h.kb, h.bad,
                                 c->flags);
            }
            if (late) HIPCHK(c, hipEventRecord(c->ev_fork, st));
            HIPCHK(c, hipStreamWaitEvent(c->side, c->ev_fork, 0));
            prologue(c->side);
            HIPCHK(c, hipEventRecord(c->ev_join, c->side));
            joined = true;
            ProfScope p(c, PHX_K_TOPK);
            launch_cert_select(st, h);
        } else {
            {
                ProfScope p(c, PHX_K_ROUTER);
                TopkOut to;
                if (fused_topk) to = TopkOut{k, D.weight_rule, L.ds, wp<int>(c, W_IDS), wp<float>(c, W_W)};
                launch_router_exact(st, T, d, E, L.wt4, rx ? x : wp<float>(c, W_RIN), wp<float>(c, W_LOGITS), to,
                                    rx ? RouterX{wp<float>(c, W_XSCALE), L.gis} : RouterX{});
            }
            if (!fused_topk) {
                ProfScope p(c, PHX_K_TOPK);
                launch_topk(st, T, E, k, D.weight_rule, wp<float>(c, W_LOGITS), L.ds, wp<int>(c, W_IDS),
                            wp<float>(c, W_W));
            }
        }
    }
    // tile sizes: the MFMA kernels' 128 (Q4_0 / Q8_0) and 32 (K-quants), the VALU kernels' 4 (their row
    // walk is VALU-bound: larger tiles cost occupancy and measured slower)
    const int tileA = mma ? kMmaTile : kmma ? kKmmaTile : kTileA;
    const int max_tiles = std::min(n, (n + tileA - 1) / tileA + E);
    {
        ProfScope p(c, PHX_K_DISPATCH);
        launch_dispatch(st, n, E, tileA, wp<int>(c, W_IDS), wp<int>(c, W_OFF), wp<int>(c, W_PERM), wp<Tile>(c, W_TILES),
                        wp<int>(c, W_NTILES));
    }
    if (joined) HIPCHK(c, hipStreamWaitEvent(st, c->ev_join, 0));  // the prologue's rows, before the products
    Act adn = make_act(c, act_fmt(D.down_type), D.down_cols, W_ADN_Q, W_ADN_D, W_ADN_S);
    if (mma || kmma) {
        adn.qh = wp<uint16_t>(c, W_ADN_H);
        adn.qhstride = D.down_cols;
    }
    adn.fold = fast && (mma || kmma);
    if (kmma && D.down_type == PHX_Q4_K) {
        adn.bh = wp<uint16_t>(c, W_ADN_BH);
        adn.bhstride = D.down_cols / 16;
    }
    {
        ProfScope p(c, PHX_K_GATE_UP);
        if (mma)  // the matrix-core gate|up also writes the down input (GELU-gated Q8_0, list order)
            launch_grouped_mfma(st, L.gu, agu, wp<Tile>(c, W_TILES), wp<int>(c, W_NTILES), max_tiles, wp<int>(c, W_PERM), k,
                                keep ? wp<float>(c, W_G) : nullptr, keep ? wp<float>(c, W_U) : nullptr, nf, nf, 0, &adn,
                                n, c->gelu_tab);
        else if (kmma)
            launch_grouped_kmma(st, L.gu, agu, wp<Tile>(c, W_TILES), wp<int>(c, W_NTILES), max_tiles, wp<int>(c, W_PERM), k,
                                wp<float>(c, W_G), wp<float>(c, W_U), nf, nf);
        else  // the down input from the product's epilogue (or k_requant right after it)
            launch_grouped(st, L.gu, agu, wp<Tile>(c, W_TILES), wp<int>(c, W_NTILES), max_tiles, tileA, wp<int>(c, W_PERM),
                           k, wp<float>(c, W_G), wp<float>(c, W_U), nf, nf, &adn, c->gelu_tab, n);
    }
    if (kmma) {
        ProfScope p(c, PHX_K_REQUANT);
        launch_requant(st, n, nf, wp<float>(c, W_G), wp<float>(c, W_U), c->gelu_tab, adn);
    }
    {
        ProfScope p(c, PHX_K_DOWN);
        if (mma)
            launch_grouped_mfma(st, L.dn, adn, wp<Tile>(c, W_TILES), wp<int>(c, W_NTILES), max_tiles, wp<int>(c, W_PERM), 1,
                                wp<float>(c, W_YD), wp<float>(c, W_YD), d, d, n);
        else if (kmma)
            launch_grouped_kmma(st, L.dn, adn, wp<Tile>(c, W_TILES), wp<int>(c, W_NTILES), max_tiles, wp<int>(c, W_PERM), 1,
                                wp<float>(c, W_YD), wp<float>(c, W_YD), d, d);
        else
            launch_grouped(st, L.dn, adn, wp<Tile>(c, W_TILES), wp<int>(c, W_NTILES), max_tiles, tileA, wp<int>(c, W_PERM),
                           1, wp<float>(c, W_YD), wp<float>(c, W_YD), d, d);
    }
    const float* sh = shared;
    if (shared_ffn) {
        ProfScope p(c, PHX_K_SHARED);
        const int nff = D.n_ff_shared;
        const int sA = smma ? kMmaTile : kTileA;
        const int smax = (T + sA - 1) / sA + 1;
        launch_dispatch(st, T, 1, sA, wp<int>(c, W_ZERO), wp<int>(c, W_SOFF), wp<int>(c, W_SPERM), wp<Tile>(c, W_STILES),
                        wp<int>(c, W_SNTILES));
        Act asd = make_act(c, act_fmt(D.shared_type), round_up(nff, block_elems(D.shared_type)), W_ASD_Q, W_ASD_D,
                           W_ASD_S);
        if (smma) {
            asd.qh = wp<uint16_t>(c, W_ASD_H);
            asd.qhstride = asd.cols;
            asd.fold = fast;
        }
        if (smma)
            launch_grouped_mfma(st, L.sgu, ash, wp<Tile>(c, W_STILES), wp<int>(c, W_SNTILES), smax, wp<int>(c, W_SPERM), 1,
                                nullptr, nullptr, nff, nff, 0, &asd, T, c->gelu_tab);  // (no reader of g, u)
        else
            launch_grouped(st, L.sgu, ash, wp<Tile>(c, W_STILES), wp<int>(c, W_SNTILES), smax, kTileA, wp<int>(c, W_SPERM),
                           1, wp<float>(c, W_SHG), wp<float>(c, W_SHU), nff, nff, &asd, c->gelu_tab, T);
        if (smma)
            launch_grouped_mfma(st, L.sdn, asd, wp<Tile>(c, W_STILES), wp<int>(c, W_SNTILES), smax, wp<int>(c, W_SPERM), 1,
                                wp<float>(c, W_SHOUT), wp<float>(c, W_SHOUT), d, d, T);
        else
            launch_grouped(st, L.sdn, asd, wp<Tile>(c, W_STILES), wp<int>(c, W_SNTILES), smax, kTileA, wp<int>(c, W_SPERM),
                           1, wp<float>(c, W_SHOUT), wp<float>(c, W_SHOUT), d, d);
        sh = wp<float>(c, W_SHOUT);
    }
    {
        ProfScope p(c, PHX_K_COMBINE);
        launch_combine(st, T, d, k, D.eps, wp<float>(c, W_YD), wp<float>(c, W_W), sh, L.post1, L.post2, out, xres,
                       L.post_ffw, c->flags);
    }
    HIPCHK(c, launch_status(c));
    return PHX_OK;
}

int run_layer(phx_moe_ctx* c, const Layer& L, int T, const float* x, const float* shared, float* out, float* xres,
              unsigned flags)
{
    if (use_decode(c, L, T, flags)) return run_layer_decode(c, L, T, x, shared, out, xres);
    return run_layer_general(c, L, T, x, shared, out, xres, (flags & PHX_FLAG_EXACT_ROUTER) != 0,
                             (flags & PHX_FLAG_FAST_MATH) != 0, (flags & PHX_FLAG_KEEP_INTERMEDIATES) != 0);
}

int upload_f32(phx_moe_ctx* c, const float* src, size_t n, float** dst)
{
    if (*dst) HIPCHK(c, hipFree(*dst));
    *dst = nullptr;
    HIPCHK(c, dev_malloc(c, (void**)dst, std::max<size_t>(n, 1) * 4));
    HIPCHK(c, hipMemcpy(*dst, src, n * 4, hipMemcpyHostToDevice));
    return PHX_OK;
}

void free_qmat(QMat& q)
{
    if (q.payload) (void)hipFree(q.payload);
    if (q.scale) (void)hipFree(q.scale);
    q.payload = nullptr;
    q.scale = nullptr;
}

constexpr size_t kIqGridBytes = 256 * 8 + 1024 * 8 + 512 * 4;

const void* iq_grid_of(const phx_moe_ctx* c, int type)
{
    if (!c->iq_grid) return nullptr;
    return type == PHX_IQ2_XXS ? c->iq_grid : type == PHX_IQ2_S ? c->iq_grid + 256 * 8 : c->iq_grid + 1280 * 8;
}

int upload_iq_grids(phx_moe_ctx* c)
{
    std::vector<uint8_t> h(kIqGridBytes);
    uint64_t* g2xxs = (uint64_t*)h.data();
    uint64_t* g2s = g2xxs + 256;
    uint32_t* g3s = (uint32_t*)(g2s + 1024);
    for (int i = 0; i < 256; i++) g2xxs[i] = phx_iq2_grid_word(phx_iq2xxs_codes[i]);
    for (int i = 0; i < 1024; i++) g2s[i] = phx_iq2_grid_word(phx_iq2s_codes[i]);
    for (int i = 0; i < 512; i++) g3s[i] = phx_iq3s_grid_word(phx_iq3s_codes[i]);
    HIPCHK(c, dev_malloc(c, (void**)&c->iq_grid, kIqGridBytes));
    HIPCHK(c, hipMemcpy(c->iq_grid, h.data(), kIqGridBytes, hipMemcpyHostToDevice));
    return PHX_OK;
}

int upload_q(phx_moe_ctx* c, int type, const void* src, int n_mat, int rows, int cols, QMat& q, bool paired = false)
{
    free_qmat(q);
    HostQ h;
    repack(type, (const uint8_t*)src, n_mat, rows, cols, q, h, paired);
    q.grid = iq_type(type) ? iq_grid_of(c, type) : nullptr;
    HIPCHK(c, dev_malloc(c, (void**)&q.payload, h.payload.size()));
    HIPCHK(c, dev_malloc(c, (void**)&q.scale, h.scale.size()));
    HIPCHK(c, hipMemcpy(q.payload, h.payload.data(), h.payload.size(), hipMemcpyHostToDevice));
    HIPCHK(c, hipMemcpy(q.scale, h.scale.data(), h.scale.size(), hipMemcpyHostToDevice));
    return PHX_OK;
}

void free_layer(Layer& L)
{
    float** fs[] = {&L.wt4, &L.wrow, &L.gis, &L.ds, &L.pre2, &L.post1, &L.post2, &L.ffn_norm, &L.post_ffw, &L.wsc, &L.wnr};
    for (float** f : fs) {
        if (*f) (void)hipFree(*f);
        *f = nullptr;
    }
    free_qmat(L.gu);
    free_qmat(L.dn);
    free_qmat(L.sgu);
    free_qmat(L.sdn);
    L.present = false;
}

void drop_graph_timing(phx_moe_ctx* c)
{
    for (auto& p : c->graph_timing) {
        (void)hipEventDestroy(p.a);
        (void)hipEventDestroy(p.b);
    }
    c->graph_timing.clear();
}

int drain_profile(phx_moe_ctx* c)
{
    if (c->pending.empty()) return PHX_OK;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    for (auto& p : c->pending) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) c->prof_ms[p.kind] += ms;
        c->pool.push_back(p.a);
        c->pool.push_back(p.b);
    }
    c->pending.clear();
    return PHX_OK;
}

}  // namespace

// One dense quantized matrix on the device (GemmaGpu's GW, src/GemmaGpu.cs:344-352), repacked into row
// groups like the experts, for phx_matmul.
struct phx_weight {
    QMat q;
    int type = 0, rows = 0, cols = 0;
};

// Workspace of phx_moe_ffn_noalloc: one array per device, which each GPU the library runs on holds
// until the process ends.  In host code the name is only a stand-in, never a device address: the
// address comes from hipGetSymbolAddress, once per device with that device current (at context
// creation), and only that address is used.  Every noalloc call on a device shares the array and
// leaves its contents behind; calls that overlap on one device race.
static __device__ __align__(256) unsigned char scratch[PHX_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
unsigned char* g_scratch_addr[kMaxDevices] = {};

// The scratch array's address on c's device (current), looked up on the device's first context.
int scratch_address(phx_moe_ctx* c)
{
    if (c->device >= kMaxDevices) return set_err(c, PHX_ERR_UNSUPPORTED, "device index %d too large", c->device);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_addr[c->device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return set_err(c, e == hipSuccess ? PHX_ERR_HIP : hip_code(e), "hipGetSymbolAddress(scratch): %s",
                           hipGetErrorString(e));
        g_scratch_addr[c->device] = (unsigned char*)p;
    }
    c->scratch = g_scratch_addr[c->device];
    return PHX_OK;
}

int check_ffn_args(phx_moe_ctx* c, int layer, int T, const float* x, float* out, unsigned flags)
{
    if (layer < 0 || layer >= (int)c->layers.size() || !c->layers[layer].present)
        return set_err(c, PHX_ERR_ARG, "layer %d not uploaded", layer);
    const Layer& L = c->layers[layer];
    if (T <= 0 || (int64_t)T * L.desc.n_used > 65535) return set_err(c, PHX_ERR_ARG, "T=%d out of range", T);
    if (!x || !out) return set_err(c, PHX_ERR_ARG, "null x/out");
    if ((flags & PHX_FLAG_RESIDUAL) && !L.post_ffw) return set_err(c, PHX_ERR_ARG, "residual needs post_ffw_norm");
    if ((flags & PHX_FLAG_RESIDUAL) && out == x) return set_err(c, PHX_ERR_ARG, "residual needs out distinct from x");
    return PHX_OK;
}

// A device-pointer call's rows must be memory the GPU can address: hipMalloc'd, managed or pinned host.
// A pageable host pointer would fault the device, so it is refused here.
bool device_accessible(const void* p)
{
    hipPointerAttribute_t at{};
    if (hipPointerGetAttributes(&at, p) != hipSuccess) {
        (void)hipGetLastError();  // the query's error is not the caller's
        return false;
    }
    return at.type == hipMemoryTypeDevice || at.type == hipMemoryTypeManaged || at.type == hipMemoryTypeHost ||
           at.type == hipMemoryTypeUnified;
}

int check_device_rows(phx_moe_ctx* c, const float* x, const float* shared, const float* out)
{
    if (!device_accessible(x)) return set_err(c, PHX_ERR_ARG, "x is not device-accessible memory");
    if (shared && !device_accessible(shared)) return set_err(c, PHX_ERR_ARG, "shared is not device-accessible memory");
    if (!device_accessible(out)) return set_err(c, PHX_ERR_ARG, "out is not device-accessible memory");
    return PHX_OK;
}

// the workspace table the last call used (routing and intermediates are read from it)
const std::vector<Buf>& last_ws(const phx_moe_ctx* c) { return c->last_scratch ? c->ws_scratch : c->ws; }

}  // namespace

// ================================================================================ C ABI

extern "C" {

int phx_moe_create(int hip_device, phx_moe_ctx** out)
{
    if (!out) return PHX_ERR_ARG;
    *out = nullptr;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) return PHX_ERR_DEVICE_LOST;
    if (hip_device < 0 || hip_device >= n) return PHX_ERR_ARG;
    phx_moe_ctx* c = new phx_moe_ctx();
    c->device = hip_device;
    if (const char* f = getenv("PHX_FAULT")) {  // "malloc:n" | "launch:n" (tests of the error paths)
        long long n = 0;
        if (sscanf(f, "malloc:%lld", &n) == 1) c->fault.site = FaultPlan::MALLOC;
        else if (sscanf(f, "launch:%lld", &n) == 1) c->fault.site = FaultPlan::LAUNCH;
        c->fault.n = n;
    }
    int rc = PHX_OK;
    do {
        hipError_t h;
        if ((h = hipSetDevice(hip_device)) != hipSuccess) { rc = set_err(c, hip_code(h), "hipSetDevice failed"); break; }
        if ((h = hipDeviceGetAttribute(&c->ncu, hipDeviceAttributeMultiprocessorCount, hip_device)) != hipSuccess) {
            rc = set_err(c, hip_code(h), "hipDeviceGetAttribute failed");
            break;
        }
        if ((h = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking)) != hipSuccess ||
            (h = hipStreamCreateWithFlags(&c->side, hipStreamNonBlocking)) != hipSuccess ||
            (h = hipEventCreateWithFlags(&c->ev_fork, hipEventDisableTiming)) != hipSuccess ||
            (h = hipEventCreateWithFlags(&c->ev_join, hipEventDisableTiming)) != hipSuccess) {
            rc = set_err(c, hip_code(h), "hipStreamCreate failed");
            break;
        }
        std::vector<float> tab;
        build_gelu_table(tab);
        if ((h = dev_malloc(c, (void**)&c->gelu_tab, tab.size() * 4)) != hipSuccess) { rc = set_err(c, hip_code(h), "OOM"); break; }
        if ((h = hipMemcpy(c->gelu_tab, tab.data(), tab.size() * 4, hipMemcpyHostToDevice)) != hipSuccess) {
            rc = set_err(c, hip_code(h), "gelu table upload failed");
            break;
        }
        if ((h = dev_malloc(c, (void**)&c->flags, 64)) != hipSuccess) { rc = set_err(c, hip_code(h), "OOM"); break; }
        if ((h = hipMemset(c->flags, 0, 64)) != hipSuccess) { rc = set_err(c, hip_code(h), "memset failed"); break; }
        if ((rc = scratch_address(c)) != PHX_OK) break;
        c->ws_scratch.resize(W_COUNT);
        if ((rc = upload_iq_grids(c)) != PHX_OK) break;
    } while (0);
    if (rc != PHX_OK) {
        phx_moe_destroy(c);
        return rc;
    }
    *out = c;
    return PHX_OK;
}

void phx_moe_destroy(phx_moe_ctx* c)
{
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    if (c->graph_exec) (void)hipGraphExecDestroy(c->graph_exec);
    if (c->graph) (void)hipGraphDestroy(c->graph);
    drop_ffn_graphs(c);
    if (c->pin) (void)hipHostFree(c->pin);
    for (auto& L : c->layers) free_layer(L);
    for (auto& b : c->ws)
        if (b.p) (void)hipFree(b.p);
    for (auto& p : c->pending) {
        (void)hipEventDestroy(p.a);
        (void)hipEventDestroy(p.b);
    }
    for (auto e : c->pool) (void)hipEventDestroy(e);
    drop_graph_timing(c);
    if (c->gelu_tab) (void)hipFree(c->gelu_tab);
    if (c->flags) (void)hipFree(c->flags);
    if (c->iq_grid) (void)hipFree(c->iq_grid);
    if (c->ev_fork) (void)hipEventDestroy(c->ev_fork);
    if (c->ev_join) (void)hipEventDestroy(c->ev_join);
    if (c->side) (void)hipStreamDestroy(c->side);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
}

const char* phx_moe_last_error(const phx_moe_ctx* c) { return c ? c->err.c_str() : "null context"; }

int phx_moe_layer_upload(phx_moe_ctx* c, int layer, const phx_moe_layer_desc* D)
{
    if (!c) return PHX_ERR_ARG;
    int rc = phx_moe_check_desc(D);
    if (rc) return set_err(c, rc, "layer %d: invalid or unsupported descriptor (%d)", layer, rc);
    if (layer < 0 || layer > 4096) return set_err(c, PHX_ERR_ARG, "layer index %d out of range", layer);
    ENTER(c);
    HIPCHK(c, hipStreamSynchronize(c->stream));
    if ((int)c->layers.size() <= layer) c->layers.resize(layer + 1);
    Layer& L = c->layers[layer];
    free_layer(L);
    L.gen = ++c->upload_gen;
    L.desc = *D;
    const int d = D->d, E = D->n_expert, nf = D->n_ff;
    // router transposed to [d/4][E][4] (consecutive experts are consecutive lanes)
    std::vector<float> wt((size_t)d * E);
    for (int e = 0; e < E; e++)
        for (int i = 0; i < d; i++) wt[((size_t)(i / 4) * E + e) * 4 + (i % 4)] = D->gate_inp[(size_t)e * d + i];
    if ((rc = upload_f32(c, wt.data(), wt.size(), &L.wt4))) return rc;
    if ((rc = upload_f32(c, D->gate_inp, (size_t)d * E, &L.wrow))) return rc;
    if ((rc = upload_f32(c, D->gate_inp_scale, d, &L.gis))) return rc;
    if (d % 16 == 0 && d / 16 >= kRouterRanges) {
        // the matrix-core router's operands: w'_i = fl(s_i w_i) (one float product, as the kernel would
        // form it) and |w'_r|^2 over each reduction range, a double sum rounded up to a float
        std::vector<float> ws((size_t)d * E), wn((size_t)E * kRouterRanges);
        for (int e = 0; e < E; e++) {
            const float* w = D->gate_inp + (size_t)e * d;
            float* o = ws.data() + (size_t)e * d;
            for (int i = 0; i < d; i++) o[i] = D->gate_inp_scale[i] * w[i];
            for (int r = 0; r < kRouterRanges; r++) {
                int c0, cnt;
                router_range(d, r, &c0, &cnt);
                double q = 0.0;
                for (int i = 16 * c0; i < 16 * (c0 + cnt); i++) q += (double)o[i] * (double)o[i];
                q *= 1.0 + 0x1p-40;  // above the double sum's relative error (n * 2^-53, n <= 4096)
                float f = (float)q;
                if ((double)f < q) f = nextafterf(f, INFINITY);
                wn[(size_t)e * kRouterRanges + r] = (q == q) ? f : NAN;
            }
        }
        if ((rc = upload_f32(c, ws.data(), ws.size(), &L.wsc))) return rc;
        if ((rc = upload_f32(c, wn.data(), wn.size(), &L.wnr))) return rc;
    }
    if ((rc = upload_f32(c, D->down_scale, E, &L.ds))) return rc;
    if ((rc = upload_f32(c, D->pre_ffw_norm_2, d, &L.pre2))) return rc;
    if ((rc = upload_f32(c, D->post_ffw_norm_1, d, &L.post1))) return rc;
    if ((rc = upload_f32(c, D->post_ffw_norm_2, d, &L.post2))) return rc;
    if (D->post_ffw_norm && (rc = upload_f32(c, D->post_ffw_norm, d, &L.post_ffw))) return rc;
    if ((rc = upload_q(c, D->gate_up_type, D->gate_up_exps, E, 2 * nf, d, L.gu, true))) return rc;
    if ((rc = upload_q(c, D->down_type, D->down_exps, E, d, D->down_cols, L.dn))) return rc;
    if (D->n_ff_shared > 0) {
        const int nff = D->n_ff_shared;
        const int64_t rb = row_bytes(D->shared_type, d);
        std::vector<uint8_t> fused((size_t)2 * nff * rb);
        memcpy(fused.data(), D->ffn_gate, (size_t)nff * rb);
        memcpy(fused.data() + (size_t)nff * rb, D->ffn_up, (size_t)nff * rb);
        if ((rc = upload_f32(c, D->ffn_norm, d, &L.ffn_norm))) return rc;
        if ((rc = upload_q(c, D->shared_type, fused.data(), 1, 2 * nff, d, L.sgu, true))) return rc;
        if ((rc = upload_q(c, D->shared_type, D->ffn_down, 1, d, round_up(nff, block_elems(D->shared_type)), L.sdn)))
            return rc;
    }
    L.present = true;
    return PHX_OK;
}

namespace {

// phx_moe_ffn on host buffers: the caller's rows pass through pinned staging rows, and the layer call,
// with the copies between the staging rows and the device rows as small kernels, is captured as a graph
// the first time a (layer, T, flags, shared given) call comes and replayed after: one graph launch and one
// wait per call (the reference records the layer once and replays the command buffer per token,
// src/GemmaGpu.cs:544-554).  A graph is kept while the layer's upload and the workspace it was captured
// over are unchanged.
int ffn_host(phx_moe_ctx* c, int layer, int T, float* x, const float* shared, float* out, unsigned flags)
{
    const Layer& L = c->layers[layer];
    const size_t bytes = (size_t)T * L.desc.d * 4;
    hipStream_t st = c->stream;
    if (c->pin_bytes < bytes) {
        HIPCHK(c, hipStreamSynchronize(st));
        drop_ffn_graphs(c);
        if (c->pin) (void)hipHostFree(c->pin);
        c->pin = nullptr;
        c->pin_bytes = 0;
        HIPCHK(c, host_malloc(c, (void**)&c->pin, 3 * bytes + 256));
        c->pin_bytes = bytes;
        // the completion word starts at zero, which the device's count never writes (pinned memory comes
        // back from the allocator with an earlier owner's bytes)
        __atomic_store_n((uint32_t*)(c->pin + 3 * (bytes / 4)), 0u, __ATOMIC_RELEASE);
    }
    float *px = c->pin, *psh = c->pin + c->pin_bytes / 4, *pout = c->pin + 2 * (c->pin_bytes / 4);
    uint32_t* done = (uint32_t*)(c->pin + 3 * (c->pin_bytes / 4));
    const bool res = flags & PHX_FLAG_RESIDUAL;
    // a decode-sized call ends with one workgroup copying the rows out and writing the completion word,
    // which the host polls (a stream wait costs more than the copies); larger calls copy with several
    // workgroups and wait on the stream
    const bool small = bytes * (res ? 2 : 1) <= (256u << 10);
    const unsigned key =
        (flags & (PHX_FLAG_RESIDUAL | PHX_FLAG_EXACT_ROUTER | PHX_FLAG_FAST_MATH | PHX_FLAG_KEEP_INTERMEDIATES)) |
        (shared ? 0x80000000u : 0u);
    std::vector<void*> sig(c->ws.size());
    for (size_t i = 0; i < c->ws.size(); i++) sig[i] = c->ws[i].p;
    hipGraphExec_t exec = nullptr;
    for (size_t i = 0; i < c->ffn_graphs.size(); i++) {
        const auto& g = c->ffn_graphs[i];
        if (g.layer == layer && g.T == T && g.key == key && g.gen == L.gen && g.ws == sig) {
            exec = g.exec;
            // least recently used last out: the hit moves to the back
            std::rotate(c->ffn_graphs.begin() + i, c->ffn_graphs.begin() + i + 1, c->ffn_graphs.end());
            break;
        }
    }
    if (exec) c->ffn_graph_hits++;
    else c->ffn_graph_misses++;
    if (!exec) {
        HIPCHK(c, hipStreamSynchronize(st));
        HIPCHK(c, hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
        float *xd = wp<float>(c, W_X), *od = wp<float>(c, W_OUT), *sd = shared ? wp<float>(c, W_SHARED) : nullptr;
        launch_copy_small(st, xd, px, (int64_t)bytes);
        if (shared) launch_copy_small(st, sd, psh, (int64_t)bytes);
        int rc = run_layer(c, L, T, xd, sd, od, res ? xd : nullptr, flags & ~PHX_FLAG_ASYNC);
        if (small) {
            launch_copy_done(st, pout, od, res ? px : nullptr, res ? xd : nullptr, (int64_t)bytes,
                             (uint32_t*)(c->flags + 15), (uint32_t*)done);
        } else {
            launch_copy_small(st, pout, od, (int64_t)bytes);
            if (res) launch_copy_small(st, px, xd, (int64_t)bytes);
        }
        const hipError_t le = launch_status(c);
        hipGraph_t g = nullptr;
        const hipError_t ce = hipStreamEndCapture(st, &g);
        if (!rc && le != hipSuccess) rc = set_err(c, hip_code(le), "%s", hipGetErrorString(le));
        if (!rc && ce != hipSuccess) rc = set_err(c, hip_code(ce), "stream capture failed: %s", hipGetErrorString(ce));
        if (!rc) {
            const hipError_t ie = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
            if (ie != hipSuccess) rc = set_err(c, hip_code(ie), "graph instantiate: %s", hipGetErrorString(ie));
        }
        if (g) (void)hipGraphDestroy(g);
        if (rc) return rc;
        // room for a few shapes per uploaded layer (prefill chunks, a partial chunk, decode); the least
        // recently used graph goes
        size_t layers_up = 0;
        for (const Layer& l : c->layers) layers_up += l.present;
        const size_t cap = std::max<size_t>(64, 4 * layers_up);
        while (c->ffn_graphs.size() >= cap) {
            (void)hipGraphExecDestroy(c->ffn_graphs.front().exec);
            c->ffn_graphs.erase(c->ffn_graphs.begin());
        }
        c->ffn_graphs.push_back(phx_moe_ctx::FfnGraph{layer, T, key, L.gen, sig, exec});
    }
    memcpy(px, x, bytes);
    if (shared) memcpy(psh, shared, bytes);
    const uint32_t before = __atomic_load_n(done, __ATOMIC_ACQUIRE);
    HIPCHK(c, hipGraphLaunch(exec, st));
    if (small) {
        // the word changes once the rows are out; a call that never ends it (a fault) is left to the stream
        // wait after two seconds, which reports the error
        const auto t0 = std::chrono::steady_clock::now();
        // the acquire load orders the reads of the output rows after the word's change
        while (__atomic_load_n(done, __ATOMIC_ACQUIRE) == before)
            if (std::chrono::steady_clock::now() - t0 > std::chrono::seconds(2)) {
                HIPCHK(c, hipStreamSynchronize(st));
                if (__atomic_load_n(done, __ATOMIC_ACQUIRE) == before) {
                    uint32_t ctr = 0;
                    (void)hipMemcpy(&ctr, c->flags + 15, 4, hipMemcpyDeviceToHost);
                    return set_err(c, PHX_ERR_HIP, "host-buffer call: no completion (word %u, device count %u)",
                                   (unsigned)__atomic_load_n(done, __ATOMIC_ACQUIRE), (unsigned)ctr);
                }
            }
    } else {
        HIPCHK(c, hipStreamSynchronize(st));
    }
    memcpy(out, pout, bytes);
    if (res) memcpy(x, px, bytes);
    c->last_T = T;
    c->last_layer = layer;
    c->last_gu_kept = keeps_gu(c, c->layers[layer], T, flags);
    return PHX_OK;
}

}  // namespace

int phx_moe_ffn(phx_moe_ctx* c, int layer, int T, float* x, const float* shared, float* out, unsigned flags)
{
    if (!c) return PHX_ERR_ARG;
    int rc = check_ffn_args(c, layer, T, x, out, flags);
    if (rc) return rc;
    const Layer& L = c->layers[layer];
    ENTER(c);
    rc = ensure_workspace(c, L, T);
    if (rc) return rc;
    c->last_scratch = false;
    const size_t bytes = (size_t)T * L.desc.d * 4;
    const bool dev = flags & PHX_FLAG_DEVICE_PTRS;
    if (dev && (rc = check_device_rows(c, x, shared, out))) return rc;
    if (!dev && !c->profiling && bytes % 16 == 0) return ffn_host(c, layer, T, x, shared, out, flags);
    float* xin = x;
    const float* shin = shared;
    float* o = out;
    if (!dev) {
        xin = wp<float>(c, W_X);
        o = wp<float>(c, W_OUT);
        HIPCHK(c, hipMemcpyAsync(xin, x, bytes, hipMemcpyHostToDevice, c->stream));
        if (shared) {
            HIPCHK(c, hipMemcpyAsync(wp<float>(c, W_SHARED), shared, bytes, hipMemcpyHostToDevice, c->stream));
            shin = wp<float>(c, W_SHARED);
        }
    }
    rc = run_layer(c, L, T, xin, shin, o, (flags & PHX_FLAG_RESIDUAL) ? xin : nullptr, flags);
    if (rc) return rc;
    c->last_T = T;
    c->last_layer = layer;
    c->last_gu_kept = keeps_gu(c, c->layers[layer], T, flags);
    if (!dev) {
        HIPCHK(c, hipMemcpyAsync(out, o, bytes, hipMemcpyDeviceToHost, c->stream));
        if (flags & PHX_FLAG_RESIDUAL) HIPCHK(c, hipMemcpyAsync(x, xin, bytes, hipMemcpyDeviceToHost, c->stream));
    }
    if (!(flags & PHX_FLAG_ASYNC) || !dev) HIPCHK(c, hipStreamSynchronize(c->stream));
    return PHX_OK;
}

int phx_moe_ffn_noalloc(phx_moe_ctx* c, int layer, int T, float* x, const float* shared, float* out, unsigned flags)
{
    if (!c) return PHX_ERR_ARG;
    int rc = check_ffn_args(c, layer, T, x, out, flags);
    if (rc) return rc;
    if (!c->scratch || (int)c->ws_scratch.size() != W_COUNT) return set_err(c, PHX_ERR_HIP, "no scratch array");
    const Layer& L = c->layers[layer];
    ENTER(c);
    if ((rc = check_device_rows(c, x, shared, out))) return rc;
    // this call's workspace table, laid out afresh inside the scratch array (no allocation: the table
    // was sized at creation and the vectors only swap)
    std::swap(c->ws, c->ws_scratch);
    for (Buf& b : c->ws) b = Buf{};
    c->bump_base = c->scratch;
    c->bump_off = 0;
    c->bump_cap = PHX_NOALLOC_SCRATCH_BYTES;
    rc = ensure_workspace(c, L, T);
    c->bump_base = nullptr;
    const bool prof = c->profiling;  // the timers would create events
    c->profiling = false;
    if (rc == PHX_OK) {
        // the shared FFN's one-expert ids must read zero; the array keeps the previous call's bytes
        if (c->ws[W_ZERO].p) launch_fill_u32(c->stream, (uint32_t*)c->ws[W_ZERO].p, (int64_t)T, 0u);
        rc = run_layer(c, L, T, x, shared, out, (flags & PHX_FLAG_RESIDUAL) ? x : nullptr, flags);
    }
    c->profiling = prof;
    std::swap(c->ws, c->ws_scratch);
    if (rc) return rc;
    HIPCHK(c, launch_status(c));
    c->last_T = T;
    c->last_layer = layer;
    c->last_gu_kept = keeps_gu(c, c->layers[layer], T, flags);
    c->last_scratch = true;
    if (!(flags & PHX_FLAG_ASYNC)) HIPCHK(c, hipStreamSynchronize(c->stream));
    return PHX_OK;
}

int phx_moe_get_routing(phx_moe_ctx* c, int32_t* ids, float* weights, int32_t* offsets, int32_t* perm, float* logits)
{
    if (!c || c->last_layer < 0) return PHX_ERR_ARG;
    const phx_moe_layer_desc& D = c->layers[c->last_layer].desc;
    const size_t n = (size_t)c->last_T * D.n_used;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    const std::vector<Buf>& ws = last_ws(c);
    if (ids) HIPCHK(c, hipMemcpy(ids, ws[W_IDS].p, n * 4, hipMemcpyDeviceToHost));
    if (weights) HIPCHK(c, hipMemcpy(weights, ws[W_W].p, n * 4, hipMemcpyDeviceToHost));
    if (offsets) HIPCHK(c, hipMemcpy(offsets, ws[W_OFF].p, (size_t)(D.n_expert + 1) * 4, hipMemcpyDeviceToHost));
    if (perm) HIPCHK(c, hipMemcpy(perm, ws[W_PERM].p, n * 4, hipMemcpyDeviceToHost));
    if (logits) HIPCHK(c, hipMemcpy(logits, ws[W_LOGITS].p, (size_t)c->last_T * D.n_expert * 4, hipMemcpyDeviceToHost));
    return PHX_OK;
}

int phx_moe_get_intermediates(phx_moe_ctx* c, float* g, float* u, float* yd)
{
    if (!c || c->last_layer < 0) return PHX_ERR_ARG;
    if ((g || u) && !c->last_gu_kept)
        return set_err(c, PHX_ERR_ARG, "the last call skipped the gate and up stores: pass PHX_FLAG_KEEP_INTERMEDIATES");
    const phx_moe_layer_desc& D = c->layers[c->last_layer].desc;
    const size_t n = (size_t)c->last_T * D.n_used;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    const std::vector<Buf>& ws = last_ws(c);
    if (g) HIPCHK(c, hipMemcpy(g, ws[W_G].p, n * D.n_ff * 4, hipMemcpyDeviceToHost));
    if (u) HIPCHK(c, hipMemcpy(u, ws[W_U].p, n * D.n_ff * 4, hipMemcpyDeviceToHost));
    if (yd) HIPCHK(c, hipMemcpy(yd, ws[W_YD].p, n * D.d * 4, hipMemcpyDeviceToHost));
    return PHX_OK;
}

// A stack of decode layers with each layer's combine folded into the next layer's router: x
// alternates between two row sets (layer i reads its x from set i % 2, the fused router of layer i + 1
// writes the new x to the other set), so no workgroup overwrites rows another still reads; the last
// layer's own combine writes the result back to W_X.  Three launches per layer and one more.
constexpr int64_t FOLD_MAX_WG = 512;

static int capture_decode_stack(phx_moe_ctx* c, int first, int n_layers, int T)
{
    hipStream_t st = c->stream;
    float* xs[2] = {wp<float>(c, W_X), wp<float>(c, W_X2)};
    float* out = wp<float>(c, W_OUT);
    DecLayerH prev{};
    for (int i = 0; i < n_layers; i++) {
        const Layer& L = c->layers[first + i];
        DecLayerH h = dec_layer(c, L, T, xs[i % 2], nullptr, out, nullptr);
        h.seq = i;
        {
            ProfScope p(c, PHX_K_ROUTER);
            if (i == 0) launch_dec_route(st, h);
            else {
                prev.xin = xs[(i - 1) % 2];
                prev.xres = xs[i % 2];
                launch_dec_route_fused(st, prev, h);
            }
        }
        {
            ProfScope p(c, PHX_K_GATE_UP);
            launch_dec_gu(st, h);
        }
        {
            ProfScope p(c, PHX_K_DOWN);
            launch_dec_down(st, h);
        }
        prev = h;
    }
    prev.xin = xs[(n_layers - 1) % 2];
    prev.xres = xs[0];
    {
        ProfScope p(c, PHX_K_COMBINE);
        launch_dec_combine(st, prev);
    }
    HIPCHK(c, launch_status(c));
    return PHX_OK;
}

int phx_moe_stack_capture(phx_moe_ctx* c, int first, int n_layers, int T)
{
    return phx_moe_stack_capture2(c, first, n_layers, T, 0);
}

int phx_moe_stack_capture2(phx_moe_ctx* c, int first, int n_layers, int T, unsigned flags)
{
    if (!c || n_layers <= 0 || first < 0 || first + n_layers > (int)c->layers.size() || T <= 0)
        return set_err(c, PHX_ERR_ARG, "bad stack range");
    ENTER(c);
    int d = c->layers[first].desc.d;
    for (int l = first; l < first + n_layers; l++) {
        const Layer& L = c->layers[l];
        if (!L.present || !L.post_ffw || L.desc.d != d) return set_err(c, PHX_ERR_ARG, "layer %d unusable in a stack", l);
        if ((int64_t)T * L.desc.n_used > 65535) return set_err(c, PHX_ERR_ARG, "T too large");
        int rc = ensure_workspace(c, L, T);
        if (rc) return rc;
    }
    if (c->graph_exec) { (void)hipGraphExecDestroy(c->graph_exec); c->graph_exec = nullptr; }
    if (c->graph) { (void)hipGraphDestroy(c->graph); c->graph = nullptr; }
    drop_graph_timing(c);
    HIPCHK(c, hipStreamSynchronize(c->stream));
    HIPCHK(c, hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal));
    c->capturing = true;  // while profiling: timing events become graph nodes around each kernel
    int rc = PHX_OK;
    // folding pays while the fused routers (T * E workgroups, two per CU by their LDS) fit the chip
    // in one round: measured on MI355X at E = 128, +7% at T = 1, +1% at T = 4, -5% at T = 8
    bool fused = n_layers > 1;
    for (int l = first; l < first + n_layers; l++)
        fused = fused && use_decode(c, c->layers[l], T, flags) && (int64_t)T * c->layers[l].desc.n_expert <= FOLD_MAX_WG;
    if (fused) rc = capture_decode_stack(c, first, n_layers, T);
    else
        for (int l = first; l < first + n_layers && rc == PHX_OK; l++)
            rc = run_layer(c, c->layers[l], T, wp<float>(c, W_X), nullptr, wp<float>(c, W_OUT), wp<float>(c, W_X), flags);
    c->capturing = false;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(c->stream, &g);
    if (rc || e != hipSuccess) drop_graph_timing(c);
    if (rc) { if (g) (void)hipGraphDestroy(g); return rc; }
    if (e != hipSuccess) return set_err(c, hip_code(e), "stream capture failed: %s", hipGetErrorString(e));
    c->graph = g;
    HIPCHK(c, hipGraphInstantiate(&c->graph_exec, g, nullptr, nullptr, 0));
    c->graph_T = T;
    c->graph_first = first;
    c->graph_n = n_layers;
    c->graph_gu_kept = keeps_gu(c, c->layers[first + n_layers - 1], T, flags);
    c->graph_gens.clear();
    for (int l = first; l < first + n_layers; l++) c->graph_gens.push_back(c->layers[l].gen);
    c->graph_ws.clear();
    for (const Buf& b : c->ws) c->graph_ws.push_back(b.p);
    return PHX_OK;
}

namespace {
// the captured stack still names live memory: no layer of it uploaded again, no workspace buffer regrown
bool stack_graph_current(const phx_moe_ctx* c)
{
    if ((int)c->graph_gens.size() != c->graph_n || c->graph_ws.size() != c->ws.size()) return false;
    for (int i = 0; i < c->graph_n; i++) {
        const int l = c->graph_first + i;
        if (l >= (int)c->layers.size() || !c->layers[l].present || c->layers[l].gen != c->graph_gens[i]) return false;
    }
    for (size_t i = 0; i < c->ws.size(); i++)
        if (c->ws[i].p != c->graph_ws[i]) return false;
    return true;
}
}  // namespace

int phx_moe_stack_run(phx_moe_ctx* c, float* x, int T, unsigned flags)
{
    if (!c || !c->graph_exec) return set_err(c, PHX_ERR_ARG, "no captured stack");
    if (T != c->graph_T || !x) return set_err(c, PHX_ERR_ARG, "T=%d differs from the captured %d", T, c->graph_T);
    if (!stack_graph_current(c))
        return set_err(c, PHX_ERR_ARG, "the captured stack is stale (a layer was uploaded again or the workspace "
                                       "grew since the capture): capture it again");
    ENTER(c);
    const size_t bytes = (size_t)T * c->layers[c->graph_first].desc.d * 4;
    const bool dev = flags & PHX_FLAG_DEVICE_PTRS;
    float* xs = wp<float>(c, W_X);
    HIPCHK(c, hipMemcpyAsync(xs, x, bytes, dev ? hipMemcpyDeviceToDevice : hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipGraphLaunch(c->graph_exec, c->stream));
    HIPCHK(c, hipMemcpyAsync(x, xs, bytes, dev ? hipMemcpyDeviceToDevice : hipMemcpyDeviceToHost, c->stream));
    c->last_T = T;
    c->last_layer = c->graph_first + c->graph_n - 1;
    c->last_gu_kept = c->graph_gu_kept;
    c->last_scratch = false;
    if (c->profiling && !c->graph_timing.empty()) {
        // a stack captured while profiling: this replay's kernel intervals, read before the next one
        HIPCHK(c, hipStreamSynchronize(c->stream));
        for (auto& p : c->graph_timing) {
            float ms = 0.0f;
            if (hipEventElapsedTime(&ms, p.a, p.b) == hipSuccess) c->prof_ms[p.kind] += ms;
            c->prof_calls[p.kind] += p.first;
        }
    }
    if (!(flags & PHX_FLAG_ASYNC) || !dev) HIPCHK(c, hipStreamSynchronize(c->stream));
    return PHX_OK;
}

int phx_moe_graph_stats(phx_moe_ctx* c, int64_t* hits, int64_t* misses)
{
    if (!c) return PHX_ERR_ARG;
    if (hits) *hits = c->ffn_graph_hits;
    if (misses) *misses = c->ffn_graph_misses;
    return PHX_OK;
}

int phx_moe_sync(phx_moe_ctx* c)
{
    if (!c) return PHX_ERR_ARG;
    ENTER(c);
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return PHX_OK;
}

int phx_moe_dev_alloc(phx_moe_ctx* c, uint64_t bytes, void** ptr)
{
    if (!c || !ptr) return PHX_ERR_ARG;
    ENTER(c);
    HIPCHK(c, dev_malloc(c, ptr, std::max<uint64_t>(bytes, 1)));
    return PHX_OK;
}

int phx_moe_dev_free(phx_moe_ctx* c, void* ptr)
{
    if (!c) return PHX_ERR_ARG;
    ENTER(c);
    HIPCHK(c, hipStreamSynchronize(c->stream));
    if (ptr) HIPCHK(c, hipFree(ptr));
    return PHX_OK;
}

int phx_moe_memcpy_h2d(phx_moe_ctx* c, void* dst, const void* src, uint64_t bytes)
{
    if (!c) return PHX_ERR_ARG;
    HIPCHK(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return PHX_OK;
}

int phx_moe_memcpy_d2h(phx_moe_ctx* c, void* dst, const void* src, uint64_t bytes)
{
    if (!c) return PHX_ERR_ARG;
    HIPCHK(c, hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream));
    HIPCHK(c, hipStreamSynchronize(c->stream));
    return PHX_OK;
}

int phx_moe_profile(phx_moe_ctx* c, int enable)
{
    if (!c) return PHX_ERR_ARG;
    int rc = drain_profile(c);
    if (rc) return rc;
    c->profiling = enable != 0;
    for (int i = 0; i < PHX_K_COUNT; i++) { c->prof_ms[i] = 0; c->prof_calls[i] = 0; }
    return PHX_OK;
}

int phx_moe_profile_read(phx_moe_ctx* c, double* total_ms, int64_t* launches)
{
    if (!c) return PHX_ERR_ARG;
    int rc = drain_profile(c);
    if (rc) return rc;
    for (int i = 0; i < PHX_K_COUNT; i++) {
        if (total_ms) total_ms[i] = c->prof_ms[i];
        if (launches) launches[i] = c->prof_calls[i];
    }
    return PHX_OK;
}

int phx_moe_selftest(phx_moe_ctx* c, int op, int n, const float* a, const float* b, float* out)
{
    if (!c || n <= 0 || !a || !b || !out || op < 0 || op > 10 || ((op == 8 || op == 9) && n % 64)) return PHX_ERR_ARG;
    int m = 0;  // op 10: the row length
    if (op == 10) {
        if (!(b[0] >= 2.0f && b[0] <= 65536.0f)) return PHX_ERR_ARG;
        m = (int)b[0];
        if ((float)m != b[0] || n % m) return PHX_ERR_ARG;
    }
    ENTER(c);
    float *da = nullptr, *db = nullptr, *dout = nullptr;
    size_t bytes = (size_t)n * 4;
    HIPCHK(c, dev_malloc(c, (void**)&da, bytes));
    HIPCHK(c, dev_malloc(c, (void**)&db, bytes));
    HIPCHK(c, dev_malloc(c, (void**)&dout, bytes));
    HIPCHK(c, hipMemcpy(da, a, bytes, hipMemcpyHostToDevice));
    HIPCHK(c, hipMemcpy(db, b, bytes, hipMemcpyHostToDevice));
    if (op == 10) launch_selftest_seq(c->stream, m, n / m, da, dout);
    else launch_selftest(c->stream, op, n, da, db, dout, c->gelu_tab);
    HIPCHK(c, hipStreamSynchronize(c->stream));
    HIPCHK(c, hipMemcpy(out, dout, bytes, hipMemcpyDeviceToHost));
    (void)hipFree(da);
    (void)hipFree(db);
    (void)hipFree(dout);
    return PHX_OK;
}

int phx_moe_stream_read(phx_moe_ctx* c, const void* buf, uint64_t bytes, int iters, double* ms)
{
    if (!c || !buf || bytes < 16 || iters <= 0 || !ms) return PHX_ERR_ARG;
    ENTER(c);
    uint32_t* sink = nullptr;
    HIPCHK(c, dev_malloc(c, (void**)&sink, 256));
    hipEvent_t a, b;
    HIPCHK(c, hipEventCreate(&a));
    HIPCHK(c, hipEventCreate(&b));
    launch_stream_read(c->stream, buf, (int64_t)bytes, sink);
    HIPCHK(c, hipEventRecord(a, c->stream));
    for (int i = 0; i < iters; i++) launch_stream_read(c->stream, buf, (int64_t)bytes, sink);
    HIPCHK(c, hipEventRecord(b, c->stream));
    HIPCHK(c, hipEventSynchronize(b));
    float t = 0.0f;
    HIPCHK(c, hipEventElapsedTime(&t, a, b));
    *ms = t / iters;
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    (void)hipFree(sink);
    return PHX_OK;
}

int phx_moe_stream_copy(phx_moe_ctx* c, void* dst, const void* src, uint64_t bytes, int iters, double* ms)
{
    if (!c || !dst || !src || bytes < 16 || bytes % 16 || iters <= 0 || !ms) return PHX_ERR_ARG;
    ENTER(c);
    hipEvent_t a = nullptr, b = nullptr;
    HIPCHK(c, hipEventCreate(&a));
    HIPCHK(c, hipEventCreate(&b));
    launch_stream_copy(c->stream, dst, src, (int64_t)bytes);
    (void)hipEventRecord(a, c->stream);
    for (int i = 0; i < iters; i++) launch_stream_copy(c->stream, dst, src, (int64_t)bytes);
    (void)hipEventRecord(b, c->stream);
    hipError_t e = hipEventSynchronize(b);
    float t = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&t, a, b);
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
    HIPCHK(c, e);
    *ms = t / iters;
    return PHX_OK;
}

int phx_moe_fallback_count(phx_moe_ctx* c, int* counts)
{
    if (!c || !counts) return PHX_ERR_ARG;
    HIPCHK(c, hipStreamSynchronize(c->stream));
    HIPCHK(c, hipMemcpy(counts, c->flags, 8, hipMemcpyDeviceToHost));
    return PHX_OK;
}

static int quant_check(phx_moe_ctx* c, int mode, const float* x, const float* aux, int rows, int n, int blk,
                       const void* qs)
{
    if (mode < PHX_QUANT_PLAIN || mode > PHX_QUANT_GELU_MUL) return set_err(c, PHX_ERR_ARG, "quant mode %d", mode);
    if (rows <= 0 || rows > 65535 || n <= 0 || n % blk)
        return set_err(c, PHX_ERR_ARG, "quant shape %d x %d (n a positive multiple of %d)", rows, n, blk);
    if (!x || !qs || (mode != PHX_QUANT_PLAIN && !aux)) return set_err(c, PHX_ERR_ARG, "quant: null buffer");
    if ((uintptr_t)x % 16 || (uintptr_t)aux % 16 || (uintptr_t)qs % 4)
        return set_err(c, PHX_ERR_ARG, "quant: x and aux need 16-byte, qs 4-byte alignment");
    return PHX_OK;
}

int phx_quant_q8_0(phx_moe_ctx* c, int mode, const float* x, const float* aux, int rows, int n, float eps, int8_t* qs,
                   uint16_t* d)
{
    if (!c) return PHX_ERR_ARG;
    int rc = quant_check(c, mode, x, aux, rows, n, 32, qs);
    if (rc) return rc;
    if (!d) return set_err(c, PHX_ERR_ARG, "quant: null buffer");
    ENTER(c);
    launch_quant(c->stream, 0, mode, rows, n, eps, x, aux, c->gelu_tab, qs, d, nullptr, nullptr, c->flags);
    HIPCHK(c, launch_status(c));
    return PHX_OK;
}

int phx_quant_q8_k(phx_moe_ctx* c, int mode, const float* x, const float* aux, int rows, int n, float eps, int8_t* qs,
                   float* d, int16_t* bsums)
{
    if (!c) return PHX_ERR_ARG;
    int rc = quant_check(c, mode, x, aux, rows, n, 256, qs);
    if (rc) return rc;
    if (!d) return set_err(c, PHX_ERR_ARG, "quant: null buffer");
    ENTER(c);
    launch_quant(c->stream, 1, mode, rows, n, eps, x, aux, c->gelu_tab, qs, nullptr, d, bsums, c->flags);
    HIPCHK(c, launch_status(c));
    return PHX_OK;
}

int phx_norm_add(phx_moe_ctx* c, float* x, const float* y, const float* w, int rows, int n, float eps, float s,
                 const float* w2, int8_t* qs, uint16_t* d)
{
    if (!c) return PHX_ERR_ARG;
    if (rows <= 0 || rows > 65535 || n <= 0 || n > 16384 || n % (w2 ? 32 : 4))
        return set_err(c, PHX_ERR_ARG, "norm_add shape %d x %d (n <= 16384, a multiple of %d)", rows, n, w2 ? 32 : 4);
    if (!x || !y || !w || (w2 && (!qs || !d))) return set_err(c, PHX_ERR_ARG, "norm_add: null buffer");
    if ((uintptr_t)x % 16 || (uintptr_t)y % 16 || (uintptr_t)w % 16 || (uintptr_t)w2 % 16 || (uintptr_t)qs % 4)
        return set_err(c, PHX_ERR_ARG, "norm_add: x, y, w, w2 need 16-byte, qs 4-byte alignment");
    ENTER(c);
    launch_norm_add(c->stream, rows, n, eps, s, x, y, w, w2, w2 ? qs : nullptr, w2 ? d : nullptr, c->flags);
    HIPCHK(c, launch_status(c));
    return PHX_OK;
}

int phx_weight_upload(phx_moe_ctx* c, int type, int rows, int cols, const void* src, phx_weight** out)
{
    if (!c || !out) return PHX_ERR_ARG;
    *out = nullptr;
    if (type != PHX_Q4_0 && type != PHX_Q8_0 && !k_type(type))
        return set_err(c, PHX_ERR_UNSUPPORTED, "weight upload: type %d (Q4_0, Q8_0, Q3_K, Q4_K, Q5_K and Q6_K only)",
                       type);
    const int be = block_elems(type);
    if (rows <= 0 || cols <= 0 || cols % be || cols > 16384 || !src)
        return set_err(c, PHX_ERR_ARG, "weight upload: shape %d x %d (cols a multiple of %d, <= 16384)", rows, cols, be);
    ENTER(c);
    HIPCHK(c, hipStreamSynchronize(c->stream));
    phx_weight* w = new phx_weight();
    w->type = type;
    w->rows = rows;
    w->cols = cols;
    const int rc = upload_q(c, type, src, 1, rows, cols, w->q, false);
    if (rc) {
        free_qmat(w->q);
        delete w;
        return rc;
    }
    *out = w;
    return PHX_OK;
}

void phx_weight_free(phx_moe_ctx* c, phx_weight* w)
{
    if (!w) return;
    if (c) {
        (void)hipSetDevice(c->device);
        (void)hipStreamSynchronize(c->stream);
    }
    free_qmat(w->q);
    delete w;
}

int phx_matmul(phx_moe_ctx* c, const phx_weight* w, int T, const int8_t* xq, const uint16_t* xd, float* y)
{
    if (!c) return PHX_ERR_ARG;
    if (!w || !xq || !xd || !y) return set_err(c, PHX_ERR_ARG, "matmul: null argument");
    if (T <= 0 || T > 65535) return set_err(c, PHX_ERR_ARG, "matmul: T=%d out of range", T);
    if (w->type != PHX_Q4_0 && w->type != PHX_Q8_0)
        return set_err(c, PHX_ERR_UNSUPPORTED, "matmul: weight type %d takes Q8_K input (phx_matmul_k)", w->type);
    if ((uintptr_t)xq % 4 || (uintptr_t)xd % 2 || (uintptr_t)y % 4)
        return set_err(c, PHX_ERR_ARG, "matmul: xq needs 4-byte, xd 2-byte, y 4-byte alignment");
    ENTER(c);
    const int nb = w->cols / 32;
    // many tokens: the matrix cores on the integers as exact fp16; a few: the VALU row walk
    const bool mma = T >= 32;
    const int A = mma ? kMmaTile : kTileA;
    const int max_tiles = (T + A - 1) / A;
    int rc;
#define ENS(id, bytes) \
    if ((rc = ensure(c, id, (size_t)(bytes)))) return rc
    ENS(W_MM_IDS, (size_t)T * 4);
    ENS(W_MM_OFF, 8);
    ENS(W_MM_PERM, (size_t)T * 4);
    ENS(W_MM_TILES, (size_t)max_tiles * sizeof(Tile));
    ENS(W_MM_NT, 4);
    ENS(W_MM_D, (size_t)T * nb * 4);
    ENS(W_MM_S, (size_t)T * nb * 4);
    if (mma) ENS(W_MM_H, (size_t)T * w->cols * 2);
#undef ENS
    hipStream_t st = c->stream;
    Act a;
    a.fmt = ACT_Q8_0;
    a.cols = w->cols;
    a.q = (int8_t*)xq;
    a.qstride = w->cols;
    a.d = wp<float>(c, W_MM_D);
    a.dstride = nb;
    a.s = wp<int>(c, W_MM_S);
    a.sstride = nb;
    if (mma) {
        a.qh = wp<uint16_t>(c, W_MM_H);
        a.qhstride = w->cols;
    }
    launch_planar_act(st, T, w->cols, xq, xd, a);
    // every token is an assignment of the one matrix: the stable dispatch gives the identity list
    launch_fill_u32(st, (uint32_t*)wp<int>(c, W_MM_IDS), T, 0u);
    launch_dispatch(st, T, 1, A, wp<int>(c, W_MM_IDS), wp<int>(c, W_MM_OFF), wp<int>(c, W_MM_PERM),
                    wp<Tile>(c, W_MM_TILES), wp<int>(c, W_MM_NT));
    if (mma)
        launch_grouped_mfma(st, w->q, a, wp<Tile>(c, W_MM_TILES), wp<int>(c, W_MM_NT), max_tiles, wp<int>(c, W_MM_PERM), 1,
                            y, y, w->rows, w->rows, 0, nullptr, 0, nullptr);
    else
        launch_grouped(st, w->q, a, wp<Tile>(c, W_MM_TILES), wp<int>(c, W_MM_NT), max_tiles, A, wp<int>(c, W_MM_PERM), 1,
                       y, y, w->rows, w->rows);
    HIPCHK(c, launch_status(c));
    return PHX_OK;
}

int phx_matmul_k(phx_moe_ctx* c, const phx_weight* w, int T, const int8_t* xq, const float* xd, float* y)
{
    if (!c) return PHX_ERR_ARG;
    if (!w || !xq || !xd || !y) return set_err(c, PHX_ERR_ARG, "matmul_k: null argument");
    if (T <= 0 || T > 65535) return set_err(c, PHX_ERR_ARG, "matmul_k: T=%d out of range", T);
    if (!k_type(w->type))
        return set_err(c, PHX_ERR_UNSUPPORTED, "matmul_k: weight type %d (Q3_K, Q4_K, Q5_K and Q6_K only)", w->type);
    if ((uintptr_t)xq % 4 || (uintptr_t)xd % 4 || (uintptr_t)y % 4)
        return set_err(c, PHX_ERR_ARG, "matmul_k: xq, xd and y need 4-byte alignment");
    ENTER(c);
    const int fmt = act_fmt(w->type), cols = w->cols;
    // the general path's rule with one matrix (at least 8 rows per matrix): the matrix cores, else the
    // VALU row walk
    const bool kmma = T >= 8 && kmma_type(w->type);
    const int A = kmma ? kKmmaTile : kTileA;
    const int max_tiles = (T + A - 1) / A;
    size_t qb, db, sb;
    act_sizes(fmt, T, cols, qb, db, sb);
    int rc;
#define ENS(id, bytes) \
    if ((rc = ensure(c, id, (size_t)(bytes)))) return rc
    ENS(W_MM_IDS, (size_t)T * 4);
    ENS(W_MM_OFF, 8);
    ENS(W_MM_PERM, (size_t)T * 4);
    ENS(W_MM_TILES, (size_t)max_tiles * sizeof(Tile));
    ENS(W_MM_NT, 4);
    ENS(W_MK_Q, qb);
    ENS(W_MM_D, db);
    ENS(W_MM_S, sb);
    if (kmma) ENS(W_MM_H, (size_t)T * cols * 2);
    if (kmma && fmt == ACT_K4) ENS(W_MK_BH, (size_t)T * (cols / 16) * 2);
#undef ENS
    hipStream_t st = c->stream;
    Act a = make_act(c, fmt, cols, W_MK_Q, W_MM_D, W_MM_S);
    if (kmma) {
        a.qh = wp<uint16_t>(c, W_MM_H);
        a.qhstride = cols;
        if (fmt == ACT_K4) {
            a.bh = wp<uint16_t>(c, W_MK_BH);
            a.bhstride = cols / 16;
        }
    }
    launch_planar_act_k(st, T, cols, xq, xd, a);
    launch_fill_u32(st, (uint32_t*)wp<int>(c, W_MM_IDS), T, 0u);
    launch_dispatch(st, T, 1, A, wp<int>(c, W_MM_IDS), wp<int>(c, W_MM_OFF), wp<int>(c, W_MM_PERM),
                    wp<Tile>(c, W_MM_TILES), wp<int>(c, W_MM_NT));
    if (kmma)
        launch_grouped_kmma(st, w->q, a, wp<Tile>(c, W_MM_TILES), wp<int>(c, W_MM_NT), max_tiles, wp<int>(c, W_MM_PERM), 1,
                            y, y, w->rows, w->rows);
    else
        launch_grouped(st, w->q, a, wp<Tile>(c, W_MM_TILES), wp<int>(c, W_MM_NT), max_tiles, A, wp<int>(c, W_MM_PERM), 1,
                       y, y, w->rows, w->rows);
    HIPCHK(c, launch_status(c));
    return PHX_OK;
}

int phx_matvec(phx_moe_ctx* c, int type, const void* w, int rows, int cols, int T, const int8_t* xq, const uint16_t* xd,
               float* y)
{
    if (!c) return PHX_ERR_ARG;
    if (type != PHX_Q4_0 && type != PHX_Q8_0)
        return set_err(c, PHX_ERR_UNSUPPORTED, "matvec: weight type %d (Q4_0 and Q8_0 only)", type);
    if (rows <= 0 || T <= 0 || T > 65535 || cols <= 0 || cols % 32 || cols > 16384)
        return set_err(c, PHX_ERR_ARG, "matvec shape %d x %d, T=%d (cols a multiple of 32, <= 16384)", rows, cols, T);
    if (!w || !xq || !xd || !y) return set_err(c, PHX_ERR_ARG, "matvec: null buffer");
    if ((uintptr_t)w % 2 || (uintptr_t)xq % 16 || (uintptr_t)xd % 2 || (uintptr_t)y % 4)
        return set_err(c, PHX_ERR_ARG, "matvec: w and xd need 2-byte, xq 16-byte, y 4-byte alignment");
    const int dev = type == PHX_Q4_0 ? PHX_Q4_0_DEV : PHX_Q8_0_DEV;
    ENTER(c);
    if (matvec_lds(dev, cols / 32) > 65536) return set_err(c, PHX_ERR_ARG, "matvec: cols %d too large", cols);
    launch_matvec(c->stream, dev, rows, cols / 32, T, (const uint8_t*)w, xq, xd, y);
    HIPCHK(c, launch_status(c));
    return PHX_OK;
}

}  // extern "C"
