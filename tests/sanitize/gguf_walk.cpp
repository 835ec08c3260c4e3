// Host driver for the sanitizer build of the GGUF reader (tests/test_gguf_sanitized.py): opens each
// file named on the command line through include/phx_gguf.h, and on success reads every key, value,
// array element (up to 64 per array), tensor and layer descriptor the API offers.  Prints one line
// per file: its return code from phx_gguf_open.  Built with -fsanitize=address,undefined, so any
// out-of-bounds read, use after free or undefined operation in gguf.cpp or desc.cpp ends the run.
#include <stdio.h>
#include <string.h>

#include "../../include/phx_gguf.h"

static void walk(phx_gguf* g)
{
    volatile int64_t sink = 0;
    const int64_t nkv = phx_gguf_n_kv(g);
    for (int64_t i = 0; i < nkv; i++) {
        const char* key = phx_gguf_key_at(g, i);
        if (!key) continue;
        int32_t at = -1;
        int64_t alen = 0, iv = 0;
        float fv = 0;
        const char* s = nullptr;
        uint64_t sl = 0;
        const int vt = phx_gguf_value_type(g, key, &at, &alen);
        sink += phx_gguf_get_int(g, key, &iv) + phx_gguf_get_float(g, key, &fv);
        if (phx_gguf_get_string(g, key, &s, &sl) == 0 && s)
            for (uint64_t j = 0; j < sl; j++) sink += s[j];
        if (vt == PHX_GGUF_ARRAY)
            for (int64_t j = 0; j < alen && j < 64; j++) {
                double dv = 0;
                sink += phx_gguf_get_array_int(g, key, j, &iv) + phx_gguf_get_array_float(g, key, j, &dv);
            }
    }
    const int64_t nt = phx_gguf_n_tensors(g);
    for (int64_t i = 0; i < nt; i++) {
        phx_gguf_tensor t;
        if (phx_gguf_tensor_at(g, i, &t) != 0) continue;
        phx_gguf_tensor u;
        sink += phx_gguf_find_tensor(g, t.name, &u);
        const unsigned char* p = (const unsigned char*)t.data;
        if (p && t.size_bytes > 0) sink += p[0] + p[t.size_bytes - 1];
    }
    phx_moe_model_config cfg;
    if (phx_gguf_moe_config(g, &cfg) == 0)
        for (int l = 0; l < cfg.n_layer && l < 8; l++)
            for (int ws = 0; ws < 2; ws++) {
                phx_moe_layer_desc d;
                sink += phx_gguf_layer_desc(g, l, ws, ws, &d);
            }
    (void)sink;
}

int main(int argc, char** argv)
{
    for (int i = 1; i < argc; i++) {
        phx_gguf* g = nullptr;
        char err[256];
        const int rc = phx_gguf_open(argv[i], &g, err, sizeof err);
        if (rc == 0) {
            walk(g);
            phx_gguf_close(g);
        }
        printf("%d\n", rc);
    }
    return 0;
}
