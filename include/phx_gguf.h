/*
 * phx_gguf.h -- C ABI of libphxmoe.so's GGUF reader: real-model ingestion for the MoE FFN layer.
 *
 * Replaces, for callers without the reference's C# host, GgufFile.Open and its validation
 * (src/Gguf.cs:92-210), the mixture-of-experts part of GemmaConfig.FromGguf (src/GemmaCpu.cs:66-74)
 * and the per-layer tensor lookup of the MoE path (src/GemmaCpu.cs:180-188, src/GemmaGpu.cs:180-188,
 * ExpertSlice src/GemmaCpu.cs:108-118).  The file is memory-mapped read-only; every data pointer
 * returned points into the mapping and stays valid until phx_gguf_close.  Host code only: no device
 * is touched, so these calls work on a machine without a GPU.  A descriptor from
 * phx_gguf_layer_desc goes to phx_moe_layer_upload, which repacks the tensors for the device
 * (the role of GemmaGpu.UploadW / UploadBlocks / UploadK, src/GemmaGpu.cs:344-436).
 */
#ifndef PHX_GGUF_H
#define PHX_GGUF_H

#include <stddef.h>
#include <stdint.h>

#include "phx_moe.h"

#ifdef __cplusplus
extern "C" {
#endif

/* A file that breaks the GGUF format or the reference's rules for it: the C# side maps this code to
 * InvalidDataException (the exception GgufFile.Load throws, src/Gguf.cs:116-210).  Missing keys and
 * tensors return PHX_ERR_ARG (KeyNotFoundException in the reference); a model that is not a Gemma MoE
 * the library can run returns PHX_ERR_UNSUPPORTED (NotSupportedException, src/GemmaCpu.cs:29,72-73). */
#define PHX_ERR_FORMAT (-6)

/* GGUF metadata value types (GgufType, src/Gguf.cs:11-15). */
#define PHX_GGUF_UINT8 0
#define PHX_GGUF_INT8 1
#define PHX_GGUF_UINT16 2
#define PHX_GGUF_INT16 3
#define PHX_GGUF_UINT32 4
#define PHX_GGUF_INT32 5
#define PHX_GGUF_FLOAT32 6
#define PHX_GGUF_BOOL 7
#define PHX_GGUF_STRING 8
#define PHX_GGUF_ARRAY 9
#define PHX_GGUF_UINT64 10
#define PHX_GGUF_INT64 11
#define PHX_GGUF_FLOAT64 12

typedef struct phx_gguf phx_gguf;

/* One tensor (GgufTensor, src/Gguf.cs:77-90): dims[0] is the contiguous (row) dimension. */
typedef struct phx_gguf_tensor {
    const char* name;  /* NUL-terminated copy, owned by the file handle */
    int32_t n_dims;
    int64_t dims[4];
    int32_t type;      /* GgmlType code (src/Gguf.cs:18-24) */
    int64_t offset;    /* relative to the data section */
    int64_t size_bytes;
    const void* data;  /* into the mapping */
} phx_gguf_tensor;

/* The mixture-of-experts model parameters GemmaConfig reads (src/GemmaCpu.cs:26-74). */
typedef struct phx_moe_model_config {
    char arch[32];             /* general.architecture: gemma4 or gemma-embedding2 */
    int32_t n_embd;            /* {arch}.embedding_length */
    int32_t n_layer;           /* {arch}.block_count */
    int32_t n_expert;          /* {arch}.expert_count */
    int32_t n_expert_used;     /* {arch}.expert_used_count */
    int32_t n_ff_exp;          /* {arch}.expert_feed_forward_length */
    float eps;                 /* {arch}.attention.layer_norm_rms_epsilon */
} phx_moe_model_config;

/* Open and validate a GGUF file (GgufFile.Open, src/Gguf.cs:107-210): magic, version 2 or 3, counts,
 * key/value pairs, general.alignment (a power of two, default 32), tensor infos (1-4 positive dims,
 * unique names), the aligned data section, and per tensor a known type, a row that is a whole number
 * of blocks, an aligned offset and bytes within the file.  On failure *out is NULL and err (when not
 * NULL) receives the reason. */
int phx_gguf_open(const char* path, phx_gguf** out, char* err, size_t err_len);
void phx_gguf_close(phx_gguf* g);
const char* phx_gguf_last_error(const phx_gguf* g);

uint32_t phx_gguf_version(const phx_gguf* g);
int64_t phx_gguf_n_tensors(const phx_gguf* g);
int64_t phx_gguf_n_kv(const phx_gguf* g);
int64_t phx_gguf_data_offset(const phx_gguf* g);
int32_t phx_gguf_alignment(const phx_gguf* g);

/* Metadata.  key_at gives the i-th key in file order (GgufFile.Keys).  value_type: the key's GgufType
 * (-1 when absent); for an array, *array_type and *array_len describe it. */
const char* phx_gguf_key_at(const phx_gguf* g, int64_t i);
int phx_gguf_value_type(const phx_gguf* g, const char* key, int32_t* array_type, int64_t* array_len);
/* GetInt / GetFloat (src/Gguf.cs:225-233): any integer, bool or float scalar, converted (a float to an
 * integer rounds half to even, as Convert.ToInt64 does; an out-of-range float is an error). */
int phx_gguf_get_int(const phx_gguf* g, const char* key, int64_t* out);
int phx_gguf_get_float(const phx_gguf* g, const char* key, float* out);
/* GetString: a pointer into the mapping and its byte length (not NUL-terminated). */
int phx_gguf_get_string(const phx_gguf* g, const char* key, const char** s, uint64_t* len);
/* Element i of an array of integers, bools or floats, converted as get_int / get_float. */
int phx_gguf_get_array_int(const phx_gguf* g, const char* key, int64_t i, int64_t* out);
int phx_gguf_get_array_float(const phx_gguf* g, const char* key, int64_t i, double* out);

/* Tensors (Tensors / TensorsByName). */
int phx_gguf_tensor_at(const phx_gguf* g, int64_t i, phx_gguf_tensor* out);
int phx_gguf_find_tensor(const phx_gguf* g, const char* name, phx_gguf_tensor* out);

/* The mixture-of-experts part of GemmaConfig.FromGguf (src/GemmaCpu.cs:26-31, 66-74): a Gemma
 * architecture, and the expert keys present because blk.0.ffn_gate_inp.weight is; at most
 * PHX_MAX_EXPERTS experts and PHX_MAX_USED used, n_ff_exp a multiple of 32. */
int phx_gguf_moe_config(const phx_gguf* g, phx_moe_model_config* out);

/* The MoE tensors of layer `layer` as a descriptor over the mapping, checked against the config
 * (src/GemmaCpu.cs:180-188): ffn_gate_inp.weight f32 [d, E], ffn_gate_inp.scale [d],
 * ffn_down_exps.scale [E], pre_ffw_norm_2 / post_ffw_norm_1 / post_ffw_norm_2 [d],
 * ffn_gate_up_exps.weight [d, 2 n_ff_exp, E] and ffn_down_exps.weight [n_ff_exp, d, E] of one
 * supported quantized type each (expert e's rows at e * rows * row bytes, ExpertSlice), post_ffw_norm
 * [d] (the layer residual's norm), and the layer's dense FFN as the shared FFN (ffn_norm [d],
 * ffn_gate / ffn_up [d, nff], ffn_down [nff, d]) unless without_shared is nonzero.  Norm tensors must
 * be f32.  weight_rule sets desc->weight_rule. */
int phx_gguf_layer_desc(const phx_gguf* g, int layer, int without_shared, int weight_rule, phx_moe_layer_desc* desc);

#ifdef __cplusplus
}
#endif
#endif
