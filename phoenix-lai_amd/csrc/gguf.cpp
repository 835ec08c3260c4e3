// GGUF reader of libphxmoe.so (include/phx_gguf.h): host code only.
//
// Follows GgufFile.Load (src/Gguf.cs:116-210): the header, key/value pairs and tensor infos are read
// with every access bounds-checked against the file length, and the reference's validation rules are
// applied in the same order with the same outcome (the reference throws InvalidDataException; here
// PHX_ERR_FORMAT with the reason).  The file is memory-mapped read-only and tensors point into the
// mapping, as GgufTensor.Data does.
#include "../../include/phx_gguf.h"

#include <fcntl.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <stdexcept>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

struct FormatError : std::runtime_error {
    using std::runtime_error::runtime_error;
};

std::string fmt(const char* f, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, f);
    vsnprintf(buf, sizeof buf, f, ap);
    va_end(ap);
    return buf;
}

struct Kv {
    std::string key;
    int32_t type = 0;
    int32_t atype = -1;   // array element type
    int64_t alen = 0;     // array length
    uint64_t pos = 0;     // file offset of the scalar value, the string's bytes, or the first array element
    uint64_t slen = 0;    // string length
};

struct Tensor {
    std::string name;
    int32_t nd = 0;
    int64_t dims[4] = {1, 1, 1, 1};
    int32_t type = 0;
    int64_t offset = 0, size = 0;
};

// Elements per block and bytes per block of a GgmlType (GgmlTypes.TryGetLayout, src/Gguf.cs:29-59).
bool layout(int32_t t, int* bs, int* ts)
{
    switch (t) {
    case 0: *bs = 1; *ts = 4; return true;      // F32
    case 1: *bs = 1; *ts = 2; return true;      // F16
    case 30: *bs = 1; *ts = 2; return true;     // BF16
    case 24: *bs = 1; *ts = 1; return true;     // I8
    case 25: *bs = 1; *ts = 2; return true;     // I16
    case 26: *bs = 1; *ts = 4; return true;     // I32
    case 27: *bs = 1; *ts = 8; return true;     // I64
    case 28: *bs = 1; *ts = 8; return true;     // F64
    case 2: *bs = 32; *ts = 18; return true;    // Q4_0
    case 3: *bs = 32; *ts = 20; return true;    // Q4_1
    case 6: *bs = 32; *ts = 22; return true;    // Q5_0
    case 7: *bs = 32; *ts = 24; return true;    // Q5_1
    case 8: *bs = 32; *ts = 34; return true;    // Q8_0
    case 9: *bs = 32; *ts = 36; return true;    // Q8_1
    case 10: *bs = 256; *ts = 84; return true;  // Q2_K
    case 11: *bs = 256; *ts = 110; return true; // Q3_K
    case 12: *bs = 256; *ts = 144; return true; // Q4_K
    case 13: *bs = 256; *ts = 176; return true; // Q5_K
    case 14: *bs = 256; *ts = 210; return true; // Q6_K
    case 15: *bs = 256; *ts = 292; return true; // Q8_K
    case 16: *bs = 256; *ts = 66; return true;  // IQ2_XXS
    case 22: *bs = 256; *ts = 82; return true;  // IQ2_S
    case 21: *bs = 256; *ts = 110; return true; // IQ3_S
    }
    return false;
}

int scalar_size(int32_t t)
{
    switch (t) {
    case PHX_GGUF_UINT8: case PHX_GGUF_INT8: case PHX_GGUF_BOOL: return 1;
    case PHX_GGUF_UINT16: case PHX_GGUF_INT16: return 2;
    case PHX_GGUF_UINT32: case PHX_GGUF_INT32: case PHX_GGUF_FLOAT32: return 4;
    case PHX_GGUF_UINT64: case PHX_GGUF_INT64: case PHX_GGUF_FLOAT64: return 8;
    }
    return 0;
}

}  // namespace

struct phx_gguf {
    int fd = -1;
    const uint8_t* base = nullptr;
    uint64_t len = 0;
    uint32_t version = 0;
    int64_t n_tensors = 0, n_kv = 0, data_off = 0;
    int32_t alignment = 32;
    std::vector<Kv> kvs;
    std::unordered_map<std::string, size_t> kv_index;
    std::vector<Tensor> tensors;
    std::unordered_map<std::string, size_t> t_index;
    std::string err;

    // ---- bounds-checked reads (GgufFile.Need and the Read* helpers, src/Gguf.cs:242-262)
    uint64_t pos = 0;
    void need(uint64_t n)
    {
        if (n > len || pos > len - n) throw FormatError("Unexpected end of GGUF header.");
    }
    template <class T>
    T rd()
    {
        need(sizeof(T));
        T v;
        memcpy(&v, base + pos, sizeof(T));
        pos += sizeof(T);
        return v;
    }
    std::string rd_string(uint64_t* at = nullptr, uint64_t* slen = nullptr)
    {
        const uint64_t n = rd<uint64_t>();
        if (n > 0x7FFFFFFFull) throw FormatError("String too long.");
        need(n);
        if (at) *at = pos;
        if (slen) *slen = n;
        std::string s((const char*)base + pos, (size_t)n);
        pos += n;
        return s;
    }
    void skip_scalar(int32_t t)
    {
        if (t == PHX_GGUF_STRING) {
            rd_string();
            return;
        }
        const int sz = scalar_size(t);
        if (!sz) throw FormatError(fmt("Unknown GGUF value type %d.", t));
        need(sz);
        pos += sz;
    }

    void load(const char* path);
    const Kv* kv(const char* key) const
    {
        auto it = kv_index.find(key);
        return it == kv_index.end() ? nullptr : &kvs[it->second];
    }
    const Tensor* tensor(const std::string& name) const
    {
        auto it = t_index.find(name);
        return it == t_index.end() ? nullptr : &tensors[it->second];
    }
};

void phx_gguf::load(const char* path)
{
    fd = ::open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) throw std::invalid_argument(fmt("cannot open %s", path));
    struct stat st;
    if (fstat(fd, &st) != 0) throw std::invalid_argument(fmt("cannot stat %s", path));
    len = (uint64_t)st.st_size;
    if (len < 24) throw FormatError("File too small to be GGUF.");
    void* m = mmap(nullptr, (size_t)len, PROT_READ, MAP_SHARED, fd, 0);
    if (m == MAP_FAILED) throw std::invalid_argument(fmt("cannot map %s", path));
    base = (const uint8_t*)m;

    if (rd<uint32_t>() != 0x46554747u) throw FormatError("Not a GGUF file (bad magic).");
    version = rd<uint32_t>();
    if (version < 2 || version > 3) throw FormatError(fmt("Unsupported GGUF version %u.", version));
    n_tensors = rd<int64_t>();
    n_kv = rd<int64_t>();
    if (n_tensors < 0 || n_kv < 0) throw FormatError("Negative tensor or KV count.");

    for (int64_t i = 0; i < n_kv; i++) {
        Kv v;
        v.key = rd_string();
        v.type = rd<int32_t>();
        if (v.type == PHX_GGUF_ARRAY) {
            v.atype = rd<int32_t>();
            v.alen = rd<int64_t>();
            if (v.alen < 0 || v.alen > 0x7FFFFFFFll) throw FormatError("Bad array length.");
            v.pos = pos;
            if (v.atype == PHX_GGUF_STRING) {
                for (int64_t j = 0; j < v.alen; j++) rd_string();
            } else {
                const int sz = scalar_size(v.atype);
                if (!sz) throw FormatError(fmt("Unsupported GGUF array type %d.", v.atype));
                const uint64_t bytes = (uint64_t)v.alen * (uint64_t)sz;
                need(bytes);
                pos += bytes;
            }
        } else if (v.type == PHX_GGUF_STRING) {
            rd_string(&v.pos, &v.slen);
        } else {
            v.pos = pos;
            skip_scalar(v.type);
        }
        if (kv_index.count(v.key)) throw FormatError("Duplicate key " + v.key + ".");
        kv_index.emplace(v.key, kvs.size());
        kvs.push_back(std::move(v));
    }

    alignment = 32;
    if (const Kv* a = kv("general.alignment")) {
        int64_t al = 0;
        if (phx_gguf_get_int(this, "general.alignment", &al) != PHX_OK || al <= 0 || al > 0xFFFFFFFFll ||
            (al & (al - 1)) != 0 || al > (1 << 30))
            throw FormatError("general.alignment must be a power of two.");
        (void)a;
        alignment = (int32_t)al;
    }

    for (int64_t i = 0; i < n_tensors; i++) {
        Tensor t;
        t.name = rd_string();
        const uint32_t nd = rd<uint32_t>();
        if (nd == 0 || nd > 4) throw FormatError(fmt("Tensor %s has %u dims.", t.name.c_str(), nd));
        t.nd = (int32_t)nd;
        for (uint32_t d = 0; d < nd; d++) {
            t.dims[d] = rd<int64_t>();
            if (t.dims[d] <= 0) throw FormatError("Tensor " + t.name + " has a non-positive dim.");
        }
        t.type = rd<int32_t>();
        t.offset = (int64_t)rd<uint64_t>();
        if (t_index.count(t.name)) throw FormatError("Duplicate tensor " + t.name + ".");
        t_index.emplace(t.name, tensors.size());
        tensors.push_back(std::move(t));
    }

    data_off = (int64_t)((pos + (uint64_t)alignment - 1) / (uint64_t)alignment * (uint64_t)alignment);

    for (Tensor& t : tensors) {
        int bs, ts;
        if (!layout(t.type, &bs, &ts))
            throw FormatError(fmt("Tensor %s uses unsupported type %d.", t.name.c_str(), t.type));
        if (t.dims[0] % bs != 0) throw FormatError("Tensor " + t.name + " row is not a multiple of the block size.");
        if (t.offset < 0 || t.offset % alignment != 0) throw FormatError("Tensor " + t.name + " offset is not aligned.");
        int64_t n = 1;
        for (int d = 0; d < t.nd; d++)
            if (__builtin_mul_overflow(n, t.dims[d], &n)) throw FormatError("Tensor " + t.name + " is too large.");
        int64_t size;
        if (__builtin_mul_overflow(n / bs, (int64_t)ts, &size)) throw FormatError("Tensor " + t.name + " is too large.");
        t.size = size;
        int64_t end;
        if (__builtin_add_overflow(data_off, t.offset, &end) || __builtin_add_overflow(end, size, &end) ||
            (uint64_t)end > len)
            throw FormatError("Tensor " + t.name + " extends past end of file.");
    }
}

namespace {

int set_err(const phx_gguf* g, int code, const std::string& msg)
{
    if (g) const_cast<phx_gguf*>(g)->err = msg;
    return code;
}

// The value of a numeric or bool scalar at p, as a double and (exactly) as an integer when integral.
bool scalar_at(const uint8_t* p, int32_t t, double* dv, int64_t* iv, bool* is_int, bool* ok_u64)
{
    *ok_u64 = true;
    switch (t) {
    case PHX_GGUF_UINT8: { uint8_t v; memcpy(&v, p, 1); *iv = v; *is_int = true; break; }
    case PHX_GGUF_INT8: { int8_t v; memcpy(&v, p, 1); *iv = v; *is_int = true; break; }
    case PHX_GGUF_BOOL: { uint8_t v; memcpy(&v, p, 1); *iv = v != 0; *is_int = true; break; }
    case PHX_GGUF_UINT16: { uint16_t v; memcpy(&v, p, 2); *iv = v; *is_int = true; break; }
    case PHX_GGUF_INT16: { int16_t v; memcpy(&v, p, 2); *iv = v; *is_int = true; break; }
    case PHX_GGUF_UINT32: { uint32_t v; memcpy(&v, p, 4); *iv = v; *is_int = true; break; }
    case PHX_GGUF_INT32: { int32_t v; memcpy(&v, p, 4); *iv = v; *is_int = true; break; }
    case PHX_GGUF_INT64: { int64_t v; memcpy(&v, p, 8); *iv = v; *is_int = true; break; }
    case PHX_GGUF_UINT64: {
        uint64_t v;
        memcpy(&v, p, 8);
        *ok_u64 = v <= 0x7FFFFFFFFFFFFFFFull;
        *iv = (int64_t)v;
        *dv = (double)v;
        *is_int = true;
        return true;
    }
    case PHX_GGUF_FLOAT32: { float v; memcpy(&v, p, 4); *dv = v; *is_int = false; return true; }
    case PHX_GGUF_FLOAT64: { double v; memcpy(&v, p, 8); *dv = v; *is_int = false; return true; }
    default: return false;
    }
    *dv = (double)*iv;
    return true;
}

int to_int(const phx_gguf* g, const char* what, const uint8_t* p, int32_t t, int64_t* out)
{
    double dv;
    int64_t iv;
    bool is_int, ok;
    if (!scalar_at(p, t, &dv, &iv, &is_int, &ok)) return set_err(g, PHX_ERR_ARG, fmt("%s is not a number", what));
    if (is_int) {
        if (!ok) return set_err(g, PHX_ERR_ARG, fmt("%s does not fit a 64-bit integer", what));
        *out = iv;
        return PHX_OK;
    }
    // Convert.ToInt64(float / double): round half to even; NaN and out-of-range values are errors
    const double r = nearbyint(dv);
    if (!(r >= -9223372036854775808.0 && r < 9223372036854775808.0))
        return set_err(g, PHX_ERR_ARG, fmt("%s does not fit a 64-bit integer", what));
    *out = (int64_t)r;
    return PHX_OK;
}

int to_double(const phx_gguf* g, const char* what, const uint8_t* p, int32_t t, double* out)
{
    double dv;
    int64_t iv;
    bool is_int, ok;
    if (!scalar_at(p, t, &dv, &iv, &is_int, &ok)) return set_err(g, PHX_ERR_ARG, fmt("%s is not a number", what));
    *out = dv;
    return PHX_OK;
}

const Kv* find_kv(const phx_gguf* g, const char* key)
{
    const Kv* v = g->kv(key);
    if (!v) set_err(g, PHX_ERR_ARG, fmt("key %s not found", key));
    return v;
}

void fill(const phx_gguf* g, const Tensor& t, phx_gguf_tensor* o)
{
    o->name = t.name.c_str();
    o->n_dims = t.nd;
    for (int d = 0; d < 4; d++) o->dims[d] = d < t.nd ? t.dims[d] : 1;
    o->type = t.type;
    o->offset = t.offset;
    o->size_bytes = t.size;
    o->data = g->base + g->data_off + t.offset;
}

}  // namespace

extern "C" {

int phx_gguf_open(const char* path, phx_gguf** out, char* err, size_t err_len)
{
    if (!out || !path) return PHX_ERR_ARG;
    *out = nullptr;
    phx_gguf* g = new phx_gguf();
    int rc = PHX_OK;
    std::string msg;
    try {
        g->load(path);
    } catch (const FormatError& e) {
        rc = PHX_ERR_FORMAT;
        msg = e.what();
    } catch (const std::exception& e) {
        rc = PHX_ERR_ARG;
        msg = e.what();
    }
    if (rc != PHX_OK) {
        if (err && err_len) snprintf(err, err_len, "%s", msg.c_str());
        phx_gguf_close(g);
        return rc;
    }
    if (err && err_len) err[0] = 0;
    *out = g;
    return PHX_OK;
}

void phx_gguf_close(phx_gguf* g)
{
    if (!g) return;
    if (g->base) munmap((void*)g->base, (size_t)g->len);
    if (g->fd >= 0) ::close(g->fd);
    delete g;
}

const char* phx_gguf_last_error(const phx_gguf* g) { return g ? g->err.c_str() : "null handle"; }
uint32_t phx_gguf_version(const phx_gguf* g) { return g ? g->version : 0; }
int64_t phx_gguf_n_tensors(const phx_gguf* g) { return g ? (int64_t)g->tensors.size() : 0; }
int64_t phx_gguf_n_kv(const phx_gguf* g) { return g ? (int64_t)g->kvs.size() : 0; }
int64_t phx_gguf_data_offset(const phx_gguf* g) { return g ? g->data_off : 0; }
int32_t phx_gguf_alignment(const phx_gguf* g) { return g ? g->alignment : 0; }

const char* phx_gguf_key_at(const phx_gguf* g, int64_t i)
{
    return g && i >= 0 && i < (int64_t)g->kvs.size() ? g->kvs[(size_t)i].key.c_str() : nullptr;
}

int phx_gguf_value_type(const phx_gguf* g, const char* key, int32_t* array_type, int64_t* array_len)
{
    if (!g || !key) return -1;
    const Kv* v = g->kv(key);
    if (!v) return -1;
    if (array_type) *array_type = v->atype;
    if (array_len) *array_len = v->alen;
    return v->type;
}

int phx_gguf_get_int(const phx_gguf* g, const char* key, int64_t* out)
{
    if (!g || !key || !out) return PHX_ERR_ARG;
    const Kv* v = find_kv(g, key);
    if (!v) return PHX_ERR_ARG;
    return to_int(g, key, g->base + v->pos, v->type, out);
}

int phx_gguf_get_float(const phx_gguf* g, const char* key, float* out)
{
    if (!g || !key || !out) return PHX_ERR_ARG;
    const Kv* v = find_kv(g, key);
    if (!v) return PHX_ERR_ARG;
    double dv;
    const int rc = to_double(g, key, g->base + v->pos, v->type, &dv);
    if (rc == PHX_OK) *out = (float)dv;
    return rc;
}

int phx_gguf_get_string(const phx_gguf* g, const char* key, const char** s, uint64_t* len)
{
    if (!g || !key || !s || !len) return PHX_ERR_ARG;
    const Kv* v = find_kv(g, key);
    if (!v) return PHX_ERR_ARG;
    if (v->type != PHX_GGUF_STRING) return set_err(g, PHX_ERR_ARG, fmt("%s is not a string", key));
    *s = (const char*)g->base + v->pos;
    *len = v->slen;
    return PHX_OK;
}

static int array_elem(const phx_gguf* g, const char* key, int64_t i, const uint8_t** p, int32_t* t)
{
    const Kv* v = find_kv(g, key);
    if (!v) return PHX_ERR_ARG;
    if (v->type != PHX_GGUF_ARRAY || v->atype == PHX_GGUF_STRING)
        return set_err(g, PHX_ERR_ARG, fmt("%s is not an array of numbers", key));
    if (i < 0 || i >= v->alen) return set_err(g, PHX_ERR_ARG, fmt("%s: index %lld out of range", key, (long long)i));
    *p = g->base + v->pos + (uint64_t)i * (uint64_t)scalar_size(v->atype);
    *t = v->atype;
    return PHX_OK;
}

int phx_gguf_get_array_int(const phx_gguf* g, const char* key, int64_t i, int64_t* out)
{
    if (!g || !key || !out) return PHX_ERR_ARG;
    const uint8_t* p;
    int32_t t;
    int rc = array_elem(g, key, i, &p, &t);
    return rc ? rc : to_int(g, key, p, t, out);
}

int phx_gguf_get_array_float(const phx_gguf* g, const char* key, int64_t i, double* out)
{
    if (!g || !key || !out) return PHX_ERR_ARG;
    const uint8_t* p;
    int32_t t;
    int rc = array_elem(g, key, i, &p, &t);
    return rc ? rc : to_double(g, key, p, t, out);
}

int phx_gguf_tensor_at(const phx_gguf* g, int64_t i, phx_gguf_tensor* out)
{
    if (!g || !out || i < 0 || i >= (int64_t)g->tensors.size()) return PHX_ERR_ARG;
    fill(g, g->tensors[(size_t)i], out);
    return PHX_OK;
}

int phx_gguf_find_tensor(const phx_gguf* g, const char* name, phx_gguf_tensor* out)
{
    if (!g || !name || !out) return PHX_ERR_ARG;
    const Tensor* t = g->tensor(name);
    if (!t) return set_err(g, PHX_ERR_ARG, fmt("tensor %s not found", name));
    fill(g, *t, out);
    return PHX_OK;
}

int phx_gguf_moe_config(const phx_gguf* g, phx_moe_model_config* out)
{
    if (!g || !out) return PHX_ERR_ARG;
    memset(out, 0, sizeof *out);
    const char* s;
    uint64_t n;
    int rc = phx_gguf_get_string(g, "general.architecture", &s, &n);
    if (rc) return rc;
    const std::string a(s, (size_t)n);
    if (a != "gemma4" && a != "gemma-embedding2") return set_err(g, PHX_ERR_UNSUPPORTED, "Not a Gemma model: " + a);
    snprintf(out->arch, sizeof out->arch, "%s", a.c_str());
    int64_t v;
    if ((rc = phx_gguf_get_int(g, (a + ".embedding_length").c_str(), &v))) return rc;
    out->n_embd = (int32_t)v;
    if ((rc = phx_gguf_get_int(g, (a + ".block_count").c_str(), &v))) return rc;
    out->n_layer = (int32_t)v;
    if ((rc = phx_gguf_get_float(g, (a + ".attention.layer_norm_rms_epsilon").c_str(), &out->eps))) return rc;
    // the MoE is detected by the first layer's router (src/GemmaCpu.cs:67)
    if (!g->tensor("blk.0.ffn_gate_inp.weight"))
        return set_err(g, PHX_ERR_UNSUPPORTED, "not a mixture-of-experts model (no blk.0.ffn_gate_inp.weight)");
    if ((rc = phx_gguf_get_int(g, (a + ".expert_count").c_str(), &v))) return rc;
    out->n_expert = (int32_t)v;
    if ((rc = phx_gguf_get_int(g, (a + ".expert_used_count").c_str(), &v))) return rc;
    out->n_expert_used = (int32_t)v;
    if ((rc = phx_gguf_get_int(g, (a + ".expert_feed_forward_length").c_str(), &v))) return rc;
    out->n_ff_exp = (int32_t)v;
    if (out->n_expert > PHX_MAX_EXPERTS || out->n_expert_used > PHX_MAX_USED || out->n_ff_exp % 32 != 0 ||
        out->n_expert <= 0 || out->n_expert_used <= 0 || out->n_expert_used > out->n_expert || out->n_ff_exp <= 0)
        return set_err(g, PHX_ERR_UNSUPPORTED, fmt("Unexpected mixture-of-experts layout (%d experts, %d used).",
                                                   out->n_expert, out->n_expert_used));
    return PHX_OK;
}

int phx_gguf_layer_desc(const phx_gguf* g, int layer, int without_shared, int weight_rule, phx_moe_layer_desc* D)
{
    if (!g || !D) return PHX_ERR_ARG;
    phx_moe_model_config c;
    int rc = phx_gguf_moe_config(g, &c);
    if (rc) return rc;
    if (layer < 0 || layer >= c.n_layer) return set_err(g, PHX_ERR_ARG, fmt("layer %d out of range", layer));
    memset(D, 0, sizeof *D);
    const std::string p = "blk." + std::to_string(layer) + ".";
    const int64_t d = c.n_embd, E = c.n_expert, nf = c.n_ff_exp;
    const Tensor* t = nullptr;
    // one tensor with the given shape; f32 when want_f32, else a quantized type
    auto get = [&](const char* name, int nd, int64_t d0, int64_t d1, int64_t d2, bool want_f32, const void** dst,
                   int32_t* type) -> int {
        t = g->tensor(p + name);
        if (!t) return set_err(g, PHX_ERR_ARG, "tensor " + p + name + " not found");
        const int64_t want[3] = {d0, d1, d2};
        int64_t n_expect = 1;
        for (int i = 0; i < nd; i++) n_expect *= want[i];
        int64_t n_have = 1;
        for (int i = 0; i < t->nd; i++) n_have *= t->dims[i];
        bool ok = n_have == n_expect;
        for (int i = 0; i < nd && i < t->nd; i++) ok = ok && t->dims[i] == want[i];
        if (!ok) return set_err(g, PHX_ERR_UNSUPPORTED, "tensor " + p + name + " has unexpected dims");
        if (want_f32 && t->type != PHX_F32) return set_err(g, PHX_ERR_UNSUPPORTED, "tensor " + p + name + " must be f32");
        *dst = g->base + g->data_off + t->offset;
        if (type) *type = t->type;
        return PHX_OK;
    };
#define GET(name, nd, a0, a1, a2, f32, dst, ty) \
    if ((rc = get(name, nd, a0, a1, a2, f32, (const void**)(dst), ty))) return rc
    GET("ffn_gate_inp.weight", 2, d, E, 1, true, &D->gate_inp, nullptr);
    GET("ffn_gate_inp.scale", 1, d, 1, 1, true, &D->gate_inp_scale, nullptr);
    GET("ffn_down_exps.scale", 1, E, 1, 1, true, &D->down_scale, nullptr);
    GET("pre_ffw_norm_2.weight", 1, d, 1, 1, true, &D->pre_ffw_norm_2, nullptr);
    GET("post_ffw_norm_1.weight", 1, d, 1, 1, true, &D->post_ffw_norm_1, nullptr);
    GET("post_ffw_norm_2.weight", 1, d, 1, 1, true, &D->post_ffw_norm_2, nullptr);
    GET("ffn_gate_up_exps.weight", 3, d, 2 * nf, E, false, &D->gate_up_exps, &D->gate_up_type);
    GET("ffn_down_exps.weight", 3, nf, d, E, false, &D->down_exps, &D->down_type);
    GET("post_ffw_norm.weight", 1, d, 1, 1, true, &D->post_ffw_norm, nullptr);
    D->d = (int32_t)d;
    D->n_expert = (int32_t)E;
    D->n_used = c.n_expert_used;
    D->n_ff = (int32_t)nf;
    D->down_cols = (int32_t)nf;  // a GGUF row is always whole blocks (validated at open)
    D->eps = c.eps;
    D->weight_rule = weight_rule;
    if (!without_shared) {
        const Tensor* fg = g->tensor(p + "ffn_gate.weight");
        if (!fg) return set_err(g, PHX_ERR_ARG, "tensor " + p + "ffn_gate.weight not found");
        const int64_t nff = fg->nd >= 2 ? fg->dims[1] : 0;
        int32_t ty_up = 0, ty_dn = 0;
        GET("ffn_norm.weight", 1, d, 1, 1, true, &D->ffn_norm, nullptr);
        GET("ffn_gate.weight", 2, d, nff, 1, false, &D->ffn_gate, &D->shared_type);
        GET("ffn_up.weight", 2, d, nff, 1, false, &D->ffn_up, &ty_up);
        GET("ffn_down.weight", 2, nff, d, 1, false, &D->ffn_down, &ty_dn);
        if (ty_up != D->shared_type || ty_dn != D->shared_type)
            return set_err(g, PHX_ERR_UNSUPPORTED, "layer " + std::to_string(layer) + ": the dense FFN's tensors differ in type");
        D->n_ff_shared = (int32_t)nff;
    }
#undef GET
    rc = phx_moe_check_desc(D);
    if (rc) return set_err(g, rc, fmt("layer %d: the library cannot run this layer's tensors (%d)", layer, rc));
    return PHX_OK;
}

}  // extern "C"
