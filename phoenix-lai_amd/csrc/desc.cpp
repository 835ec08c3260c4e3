// Descriptor validation (host C++, no device code): shared by the library and by the GGUF reader's
// sanitizer build, which links this file and gguf.cpp alone.
#include "../../include/phx_moe.h"

namespace {
bool iq_desc_type(int t) { return t == PHX_IQ2_XXS || t == PHX_IQ2_S || t == PHX_IQ3_S; }
bool quant_type(int t)
{
    return t == PHX_Q4_0 || t == PHX_Q8_0 || t == PHX_Q3_K || t == PHX_Q4_K || t == PHX_Q5_K || t == PHX_Q6_K ||
           iq_desc_type(t);
}
int block_elems(int t) { return (t == PHX_Q4_0 || t == PHX_Q8_0) ? 32 : 256; }
int round_up(int v, int m) { return (v + m - 1) / m * m; }
}  // namespace

extern "C" int phx_moe_check_desc(const phx_moe_layer_desc* D)
{
    if (!D) return PHX_ERR_ARG;
    if (D->d <= 0 || D->n_expert <= 0 || D->n_used <= 0 || D->n_ff <= 0) return PHX_ERR_ARG;
    if (D->n_expert > PHX_MAX_EXPERTS || D->n_used > PHX_MAX_USED || D->n_used > D->n_expert) return PHX_ERR_UNSUPPORTED;
    if (D->n_ff % 32 != 0 || D->d % 32 != 0) return PHX_ERR_UNSUPPORTED;
    if (!quant_type(D->gate_up_type) || !quant_type(D->down_type)) return PHX_ERR_UNSUPPORTED;
    if (D->d % block_elems(D->gate_up_type) != 0) return PHX_ERR_UNSUPPORTED;
    if (D->down_cols != round_up(D->n_ff, block_elems(D->down_type))) return PHX_ERR_ARG;
    if (D->weight_rule != PHX_WEIGHTS_SOFTMAX && D->weight_rule != PHX_WEIGHTS_CPUREF) return PHX_ERR_ARG;
    if (!D->gate_inp || !D->gate_inp_scale || !D->down_scale || !D->pre_ffw_norm_2 || !D->post_ffw_norm_1 ||
        !D->post_ffw_norm_2 || !D->gate_up_exps || !D->down_exps)
        return PHX_ERR_ARG;
    if (!(D->eps >= 0.0f)) return PHX_ERR_ARG;
    if (D->n_ff_shared < 0) return PHX_ERR_ARG;
    if (D->n_ff_shared > 0) {
        if (!quant_type(D->shared_type)) return PHX_ERR_UNSUPPORTED;
        if (D->d % block_elems(D->shared_type) != 0 || D->n_ff_shared % 32 != 0) return PHX_ERR_UNSUPPORTED;
        if (block_elems(D->shared_type) == 256 && D->n_ff_shared % 256 != 0) return PHX_ERR_UNSUPPORTED;
        if (!D->ffn_norm || !D->ffn_gate || !D->ffn_up || !D->ffn_down) return PHX_ERR_ARG;
    }
    return PHX_OK;
}
