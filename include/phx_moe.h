/*
 * phx_moe.h -- C ABI of libphxmoe.so, the MI355X (gfx950) mixture-of-experts FFN layer of
 * phoenix-lai's Gemma 4 26B-A4B path.
 *
 * The library replaces, for this path only, the Vulkan device layer that GemmaGpu's three MoE call
 * sites record into (src/Gpu.cs:566 CreateKernel, src/Gpu.cs:848-867 Record):
 *   GemmaGpu.RecordMoe      (src/GemmaGpu.cs:656-669)  -> phx_moe_ffn, T = 1, shared given
 *   GemmaGpu.RecordFfnMoe   (src/GemmaGpu.cs:683-704)  -> phx_moe_ffn, T = 1, shared FFN computed
 *   GemmaGpu.RecordMoeRows  (src/GemmaGpu.cs:850-882)  -> phx_moe_ffn, T rows
 * and computes what GemmaCpu.MoeFfn (src/GemmaCpu.cs:376-422) defines, with the same rounding:
 * router ids and per-expert lists are bit-exact, outputs match the CPU reference to the last bit
 * except where the reference's libm (exp) rounds differently.
 *
 * Plain pointers and sizes only.  One context is used by one thread at a time (the C# host keeps
 * GpuGate.Lock, src/Vulkan.cs:210-215).  Host buffers are borrowed for the duration of a call.
 */
#ifndef PHX_MOE_H
#define PHX_MOE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Return codes.  The C# side maps PHX_ERR_DEVICE_LOST to GpuDeviceLostException
 * (src/Vulkan.cs:194-208), PHX_ERR_ARG to ArgumentException (src/Gpu.cs:851-852) and
 * PHX_ERR_UNSUPPORTED to NotSupportedException (src/GemmaGpu.cs:189-190, src/GemmaCpu.cs:72-73). */
#define PHX_OK 0
#define PHX_ERR_ARG (-1)
#define PHX_ERR_OOM (-2)
#define PHX_ERR_UNSUPPORTED (-3)
#define PHX_ERR_DEVICE_LOST (-4)
#define PHX_ERR_HIP (-5)

/* GgmlType codes of the supported tensors (src/Gguf.cs:18-24). */
#define PHX_F32 0
#define PHX_Q4_0 2
#define PHX_Q8_0 8
#define PHX_Q3_K 11 /* 110 B / 256: hmask, 2-bit q, 16 six-bit scales, d (src/CpuRefIQuants.cs:9, 19-43) */
#define PHX_Q4_K 12
#define PHX_Q5_K 13 /* 176 B / 256: Q4_K with a fifth bit per value from qh[32] (src/CpuRefKQuants.cs:13, 134-146) */
#define PHX_Q6_K 14
/* IQ expert formats (CpuRefIQuants.cs:9-12: 256-element super-blocks of 66, 82 and 110 bytes), dotted
 * against Q8_K activations by the reference's DotIQ2XXS / DotIQ2S / DotIQ3S (src/CpuRefIQuants.cs:45-167)
 * with the codebooks of src/IqTables.cs. */
#define PHX_IQ2_XXS 16
#define PHX_IQ3_S 21
#define PHX_IQ2_S 22

/* Layout limits of the reference (src/KernelsMoe.cs:43, checked at src/GemmaCpu.cs:72-73). */
#define PHX_MAX_EXPERTS 256
#define PHX_MAX_USED 16

/* Router weight rule.  PHX_WEIGHTS_SOFTMAX: renormalised softmax over the k selected logits
 * (src/KernelsMoe.cs:80-98; llama.cpp build_moe_ffn), evaluated with GemmaCpu's double exp/sum.
 * PHX_WEIGHTS_CPUREF: GemmaCpu.cs:406-407 as written, whose in-place update of sel[0] turns every
 * later term into exp(l_j - 1). */
#define PHX_WEIGHTS_SOFTMAX 0
#define PHX_WEIGHTS_CPUREF 1

/* phx_moe_ffn flags */
#define PHX_FLAG_DEVICE_PTRS 1u /* x, shared, out are device pointers (no PCIe copies) */
#define PHX_FLAG_ASYNC 2u       /* return after enqueueing; phx_moe_sync waits */
#define PHX_FLAG_RESIDUAL 4u    /* also x += rmsnorm(out) * post_ffw_norm (src/GemmaCpu.cs:355-356); x is updated in place
                                   and out must not be x */
#define PHX_FLAG_EXACT_ROUTER 8u /* replay the reference's float router sums for every token (logits, weights and
                                    outputs bit-exact to the CPU reference) instead of the certified routers
                                    (the default: sums with error bounds, the reference's float chains only for
                                    the tokens whose top-k order the bounds leave open; ids and lists are the
                                    reference's either way, logits and weights then within ~1e-6 of them) */
#define PHX_FLAG_FAST_MATH 16u /* tolerance mode of the prefill-sized expert products on the matrix cores
                                  (Q4_0 / Q8_0 and Q4_K / Q6_K; the role of the reference's f16 cooperative-
                                  matrix path, src/KernelsCoop.cs:1-10, src/GemmaGpu.cs:893): block scales folded
                                  into fp16 operands and whole rows accumulated on the matrix cores.  Routing,
                                  ids and lists are unchanged (bit-exact); the products differ from the CPU
                                  reference's chains by the operands' fp16 rounding, and the GELU-gated requant
                                  amplifies that where a value sits near a rounding boundary.  Decode-sized
                                  calls ignore it. */
#define PHX_FLAG_KEEP_INTERMEDIATES 32u /* also store the gate and up products for phx_moe_get_intermediates
                                           (debug; no counterpart in the reference).  The prefill-sized Q4_0 /
                                           Q8_0 expert products feed their GELU-gated requant straight into the
                                           down product and skip those stores without it. */

typedef struct phx_moe_ctx phx_moe_ctx;

/* One MoE layer as the GGUF file holds it (tensor names from src/GemmaCpu.cs:180-188; GGUF dims
 * list ne[0] first, src/Gguf.cs:77-90):
 *   gate_inp        ffn_gate_inp.weight     f32  [d, E]          -> E rows of d
 *   gate_inp_scale  ffn_gate_inp.scale      f32  [d]
 *   down_scale      ffn_down_exps.scale     f32  [E]
 *   pre_ffw_norm_2, post_ffw_norm_1, post_ffw_norm_2   f32 [d]
 *   gate_up_exps    ffn_gate_up_exps.weight quant [d, 2nf, E]   -> per expert 2nf rows (gate, then up)
 *   down_exps       ffn_down_exps.weight    quant [down_cols, d, E]
 * down_cols is n_ff for Q4_0/Q8_0 and n_ff rounded up to 256 for K-quants: the rows are
 * zero-padded, an extension (the reference refuses such rows, src/Gguf.cs:202-203).
 * Optional dense shared FFN (n_ff_shared > 0; src/GemmaCpu.cs:348-353): ffn_norm [d],
 * ffn_gate/ffn_up [d, n_ff_shared], ffn_down [n_ff_shared, d], all of shared_type.
 * post_ffw_norm [d] is the layer's post-FFN norm, needed only with PHX_FLAG_RESIDUAL. */
typedef struct phx_moe_layer_desc {
    int32_t d;
    int32_t n_expert;
    int32_t n_used;
    int32_t n_ff;
    int32_t down_cols;
    float eps;
    int32_t gate_up_type;
    int32_t down_type;
    int32_t weight_rule;
    int32_t n_ff_shared;
    int32_t shared_type;
    int32_t reserved;
    const float* gate_inp;
    const float* gate_inp_scale;
    const float* down_scale;
    const float* pre_ffw_norm_2;
    const float* post_ffw_norm_1;
    const float* post_ffw_norm_2;
    const void* gate_up_exps;
    const void* down_exps;
    const float* ffn_norm;
    const void* ffn_gate;
    const void* ffn_up;
    const void* ffn_down;
    const float* post_ffw_norm;
} phx_moe_layer_desc;

/* Context: device, stream, all device memory.  Replaces GpuDevice.Create (src/Gpu.cs:255). */
int phx_moe_create(int hip_device, phx_moe_ctx** out);
void phx_moe_destroy(phx_moe_ctx* ctx);
const char* phx_moe_last_error(const phx_moe_ctx* ctx);

/* Shape and type validation of a descriptor, without touching the GPU (the checks of
 * src/GemmaCpu.cs:72-73 and src/GemmaGpu.cs:189-190 generalised to the supported types). */
int phx_moe_check_desc(const phx_moe_layer_desc* desc);

/* Upload (and repack) one layer's tensors from host memory; replaces GemmaGpu's MoE uploads
 * (src/GemmaGpu.cs:178-192 UploadF32/UploadW, repack src/GemmaGpu.cs:340-436).  Layers are indexed
 * from 0; uploading an index again replaces it. */
int phx_moe_layer_upload(phx_moe_ctx* ctx, int layer, const phx_moe_layer_desc* desc);

/* One MoE FFN block for T token rows (src/GemmaGpu.cs:656-704 for T = 1, :850-882 for T rows):
 *   out[t] = rmsnorm(shared[t]) * post_ffw_norm_1 + rmsnorm(sum_j w_tj * down_e(gelu(gate_e(n)) * up_e(n))) * post_ffw_norm_2
 * with n = rmsnorm(x[t]) * pre_ffw_norm_2 and (e, w) the router's top-k.  shared == NULL: the
 * layer's shared FFN is computed from x when it has one, else the shared branch is zero.
 * x, shared: [T][d] f32; out: [T][d] f32. */
int phx_moe_ffn(phx_moe_ctx* ctx, int layer, int T, float* x, const float* shared, float* out, unsigned flags);

/* phx_moe_ffn without allocating: no counterpart in the reference.  For callers that cannot allocate
 * device memory (tight serving loops, harnesses that forbid hipMalloc).  The work runs on the context's
 * own stream, so a graph capture on a caller's stream does not record it.
 * The same computation and kernels as phx_moe_ffn with PHX_FLAG_DEVICE_PTRS (x, shared, out must be
 * device-accessible memory: hipMalloc'd, managed or pinned host; a pageable host pointer returns
 * PHX_ERR_ARG; PHX_FLAG_RESIDUAL, PHX_FLAG_EXACT_ROUTER and PHX_FLAG_ASYNC apply), but the call's workspace
 * (activations, routing, lists, intermediates) lives in a fixed array of PHX_NOALLOC_SCRATCH_BYTES per
 * device instead of the context's arena, and the call makes no hipMalloc / hipFree.  A call whose
 * workspace would not fit returns PHX_ERR_ARG (at C2's shapes every T up to 64 fits).  Every noalloc
 * call on one device shares that array and leaves its contents behind: calls that overlap on one
 * device (several contexts or threads) race.  Profiling timers are not applied. */
#define PHX_NOALLOC_SCRATCH_BYTES (32u << 20)
int phx_moe_ffn_noalloc(phx_moe_ctx* ctx, int layer, int T, float* x, const float* shared, float* out,
                        unsigned flags);

/* Routing of the last phx_moe_ffn call (any pointer may be NULL): ids [T][k] best first,
 * weights [T][k] (with ffn_down_exps.scale folded in, src/GemmaCpu.cs:417), offsets [E+1] and
 * perm [T*k] (expert e's assignments a = t*k + j in ascending order: perm[offsets[e]..offsets[e+1]),
 * the lists of src/KernelsMoe.cs:281-330), logits [T][E]. */
int phx_moe_get_routing(phx_moe_ctx* ctx, int32_t* ids, float* weights, int32_t* offsets, int32_t* perm, float* logits);

/* Expert intermediates of the last call (debug; NULL skips): g, u [T*k][n_ff] gate/up products
 * and yd [T*k][d] the down products, in assignment order a = t*k + j.  g and u of a prefill-sized
 * Q4_0 / Q8_0 call are kept only with PHX_FLAG_KEEP_INTERMEDIATES: asking for them after a call that
 * skipped them returns PHX_ERR_ARG. */
int phx_moe_get_intermediates(phx_moe_ctx* ctx, float* g, float* u, float* yd);

/* Consecutive layers as one HIP graph (batched decode): each layer does phx_moe_ffn with
 * PHX_FLAG_RESIDUAL on a device-resident x of T rows.  capture once, then run many times. */
int phx_moe_stack_capture(phx_moe_ctx* ctx, int first_layer, int n_layers, int T);
/* The same with phx_moe_ffn flags applied to every layer (PHX_FLAG_EXACT_ROUTER). */
int phx_moe_stack_capture2(phx_moe_ctx* ctx, int first_layer, int n_layers, int T, unsigned flags);
/* Replays the captured stack.  Returns PHX_ERR_ARG when a layer of the stack was uploaded again or the
 * workspace grew (a larger phx_moe_ffn call) since the capture: the graph would name freed memory, so
 * the caller captures again. */
int phx_moe_stack_run(phx_moe_ctx* ctx, float* x_inout, int T, unsigned flags);

int phx_moe_sync(phx_moe_ctx* ctx);

/* Host-buffer calls of phx_moe_ffn replay a graph captured per (layer, T, flags, shared given); this
 * returns how many calls found their graph and how many captured one (no counterpart in the reference:
 * the graph cache is this library's).  The cache keeps the least recently used graphs out first, with
 * room for four shapes per uploaded layer (at least 64). */
int phx_moe_graph_stats(phx_moe_ctx* ctx, int64_t* hits, int64_t* misses);

/* Device memory for callers without their own allocator (test harness, benchmark). */
int phx_moe_dev_alloc(phx_moe_ctx* ctx, uint64_t bytes, void** ptr);
int phx_moe_dev_free(phx_moe_ctx* ctx, void* ptr);
int phx_moe_memcpy_h2d(phx_moe_ctx* ctx, void* dst, const void* src, uint64_t bytes);
int phx_moe_memcpy_d2h(phx_moe_ctx* ctx, void* dst, const void* src, uint64_t bytes);

/* Per-kernel timing on the library's stream (the Gpu.cs:163-171 profiling counterpart).  While
 * enabled, every kernel is launched with start/stop events stamped with its own execution interval
 * (hipExtLaunchKernel), the interval a kernel-trace profiler reports.  A stack captured while
 * profiling holds the events as graph nodes around each kernel (the interval from the previous node's
 * end to the kernel's end); each phx_moe_stack_run of it then waits for the replay and adds them up.
 * profile_read returns, per kind, the summed kernel time (ms) and the number of launches of that
 * kind.  Kinds: */
#define PHX_K_PROLOGUE 0
#define PHX_K_ROUTER 1
#define PHX_K_TOPK 2
#define PHX_K_DISPATCH 3
#define PHX_K_GATE_UP 4
#define PHX_K_REQUANT 5
#define PHX_K_DOWN 6
#define PHX_K_COMBINE 7
#define PHX_K_SHARED 8
#define PHX_K_COUNT 9
int phx_moe_profile(phx_moe_ctx* ctx, int enable);
int phx_moe_profile_read(phx_moe_ctx* ctx, double* total_ms, int64_t* launches);

/* Arithmetic self-test: runs the library's device primitives on n host inputs so a test can check
 * them bit for bit against IEEE results.  op: 0 f32 division a/b, 1 rms scale 1/(float)sqrt(a+b)
 * as the reference writes it, 2 double->float of (double)a/(double)b, 3 roundf(a), 4 fp16 bits of a
 * (round to nearest even), 5 nearest-even int of a (1.5*2^23 trick), 6 GELU(a), 7 the float of
 * fp16 bits a; 8 and 9 one fp32 matrix-core product (v_mfma_f32_16x16x4_f32) per 64 inputs (n a
 * multiple of 64): lane l of a group supplies A[l % 16][l / 16] = a and B[l / 16][l % 16] = b, the
 * accumulator starts at 0 (8) or 1 (9), and out holds D[4 (l / 16)][l % 16] (the numerics the
 * many-token router's error bound assumes); 10 the sequential double sum of squares of each row of
 * m = b[0] floats of a (n a multiple of m, 2 <= m <= 65536), the sum RmsNorm's certified means fall back
 * to, formed by one wave as the kernels form it: out[2 r] and out[2 r + 1] hold the low and high 32
 * bits of row r's double.  out is float (int results as their value). */
int phx_moe_selftest(phx_moe_ctx* ctx, int op, int n, const float* a, const float* b, float* out);

/* Average time (ms) of `iters` coalesced streaming reads of a device buffer: the achievable HBM
 * read rate that the roofline figures are compared with (no counterpart in the reference). */
int phx_moe_stream_read(phx_moe_ctx* ctx, const void* buf, uint64_t bytes, int iters, double* ms);

/* Average time (ms) of `iters` streaming copies of `bytes` (a multiple of 16) between two device
 * buffers: a kernel of known traffic for scaling a profiler's memory counters (no counterpart in the
 * reference). */
int phx_moe_stream_copy(phx_moe_ctx* ctx, void* dst, const void* src, uint64_t bytes, int iters, double* ms);

/* Fallbacks since the context was created (counts[2]): [0] row norms whose double sum of squares
 * could not be certified to round like the reference's sequential sum (re-summed sequentially),
 * [1] decode-path tokens whose top-k order could not be certified (router re-run as the
 * reference's float chains). */
int phx_moe_fallback_count(phx_moe_ctx* ctx, int* counts);

/* Activation quantizers, the standalone form of KernelsQuant.Q80 / KernelsQuant.Q8K
 * (src/KernelsQuant.cs:57-172) as GemmaGpu.Quant / Q80To record them (src/GemmaGpu.cs:442-461,
 * 670-677).  Each of `rows` rows of n floats at x is quantized like CpuRef.QuantizeQ8_0
 * (src/CpuRef.cs:49-62) or CpuRef.QuantizeQ8_K (src/CpuRefKQuants.cs:53-86) applied to
 *   PHX_QUANT_PLAIN     x
 *   PHX_QUANT_SILU_MUL  silu(x) * aux        (CpuRef.Silu, src/CpuRef.cs:225-228; aux rows x n)
 *   PHX_QUANT_RMS_NORM  CpuRef.RmsNorm(x, aux, eps) per row (src/CpuRef.cs:183-191; aux [n])
 *   PHX_QUANT_GELU_MUL  gelu(x) * aux        (src/CpuRefGemma.cs:85-92; aux rows x n)
 * into CpuRef.Q8Activations' planar layout (src/CpuRef.cs:34-46): qs int8 [rows][n]; Q8_0 d fp16 bits
 * [rows][n/32]; Q8_K d float [rows][n/256] and bsums int16 [rows][n/16] (bsums may be null).
 * Device pointers (x and aux 16-byte aligned, qs 4-byte aligned); n a multiple of 32 (Q8_K: 256);
 * asynchronous on the context's stream (phx_moe_sync waits).  No counterpart takes several rows in
 * the reference; one row is its case. */
#define PHX_QUANT_PLAIN 0
#define PHX_QUANT_SILU_MUL 1
#define PHX_QUANT_RMS_NORM 2
#define PHX_QUANT_GELU_MUL 3
int phx_quant_q8_0(phx_moe_ctx* ctx, int mode, const float* x, const float* aux, int rows, int n, float eps,
                   int8_t* qs, uint16_t* d);
int phx_quant_q8_k(phx_moe_ctx* ctx, int mode, const float* x, const float* aux, int rows, int n, float eps,
                   int8_t* qs, float* d, int16_t* bsums);

/* Residual norm-add with the next norm's quantized input: KernelsGemma.NormAdd (w2 null) and
 * NormAddQuant (src/KernelsGemma.cs:126-226), recorded at src/GemmaGpu.cs:614 and 644 (the router's
 * and the next layer's input producers).  Per row of n: x = x + CpuRef.RmsNorm(y, w, eps), then
 * x *= s when s != 1 (GemmaCpu.PostAndFfn, src/GemmaCpu.cs:353-356, 367); with w2, qs / d get the
 * Q8_0 quantization of CpuRef.RmsNorm(x, w2, eps) (src/CpuRef.cs:49-62, 183-191) in the layout of
 * phx_quant_q8_0.  Device pointers (x, y, w, w2 16-byte aligned); n <= 16384, a multiple of 4 (32
 * with w2); asynchronous on the context's stream. */
int phx_norm_add(phx_moe_ctx* ctx, float* x, const float* y, const float* w, int rows, int n, float eps, float s,
                 const float* w2, int8_t* qs, uint16_t* d);

/* Dense matvec of quantized weights: KernelsGemma.MatVecQ4_0 and the Q8_0 matvec as GemmaGpu.MatVec
 * records them (src/KernelsGemma.cs:244-306, src/GemmaGpu.cs:463-476); the shared FFN's projections
 * are its callers.  w: `rows` GGUF rows of `cols` (type PHX_Q4_0 or PHX_Q8_0, row r at r * row bytes,
 * as the file holds them).  xq / xd: T Q8_0 input rows in the layout of phx_quant_q8_0.  y[t][r] is
 * CpuRef.MatVec's value (src/CpuRef.cs:91-119, src/CpuRefGemma.cs:12-40: the block terms
 * (float)isum * (d_w * d_x) added in block order).  Device pointers (xq 16-byte aligned); cols a
 * multiple of 32, at most
 * 16384 (Q8_0: 13,792); other weight types return PHX_ERR_UNSUPPORTED. */
int phx_matvec(phx_moe_ctx* ctx, int type, const void* w, int rows, int cols, int T, const int8_t* xq,
               const uint16_t* xd, float* y);

/* Prefill matmul of a dense quantized matrix over T token rows: KernelsPrefill.MatMulQ4Q8Tile as
 * GemmaGpu.Mm records it (src/KernelsPrefill.cs:143-260, src/GemmaGpu.cs:907-923) for the shared FFN
 * and every other dense projection of a prompt chunk.  phx_weight_upload repacks `rows` GGUF rows of
 * `cols` (PHX_Q4_0 or PHX_Q8_0; PHX_Q3_K, PHX_Q4_K, PHX_Q5_K or PHX_Q6_K for phx_matmul_k, cols a multiple of 256; host
 * memory, as the file holds them) into the device's row groups once (GemmaGpu.UploadW / UploadK,
 * src/GemmaGpu.cs:344-352, 402-436); phx_weight_free releases them.  phx_matmul: xq / xd are
 * T Q8_0 rows in the layout of phx_quant_q8_0 (device pointers, xq 4-byte aligned) and
 * y[t][r] = CpuRef.MatVec's value for token t (src/CpuRef.cs:91-119, src/CpuRefGemma.cs:12-40: the block
 * terms (float)isum * (d_w * d_x) added in block order), on the matrix cores for T >= 32;
 * asynchronous on the context's stream.  cols a multiple of 32, at most 16384. */
typedef struct phx_weight phx_weight;
int phx_weight_upload(phx_moe_ctx* ctx, int type, int rows, int cols, const void* gguf_rows, phx_weight** out);
void phx_weight_free(phx_moe_ctx* ctx, phx_weight* w);
int phx_matmul(phx_moe_ctx* ctx, const phx_weight* w, int T, const int8_t* xq, const uint16_t* xd, float* y);

/* Dense K-quant matvec over T token rows: KernelsK.MatVec for Q4_K / Q5_K / Q6_K weights as GemmaGpu.MatVec
 * records it (src/KernelsKQuants.cs:65-108, src/GemmaGpu.cs:471-473, bindings w, kq, kd, y), and Q3_K
 * rows as CpuRef.MatVec computes them (src/CpuRef.cs:79-85), for any K-quant dense projection (the shared
 * FFN and attention of a K-quant model).  w: a phx_weight_upload handle of a K-quant type (cols a
 * multiple of 256; Q4_0 / Q8_0 handles return
 * PHX_ERR_UNSUPPORTED).  xq / xd: T Q8_K input rows in the layout of phx_quant_q8_k (qs int8 [T][cols],
 * d float [T][cols/256]; device pointers, 4-byte aligned); the block sums are formed from xq.
 * y[t][r] = CpuRefKQuants.MatVecK's value for token t (src/CpuRefKQuants.cs:176-232: DotK's integer lane
 * sums, the eight float lanes and their fold); on the matrix cores from 8 rows, the VALU row walk below;
 * asynchronous on the context's stream. */
int phx_matmul_k(phx_moe_ctx* ctx, const phx_weight* w, int T, const int8_t* xq, const float* xd, float* y);

#ifdef __cplusplus
}
#endif
#endif
