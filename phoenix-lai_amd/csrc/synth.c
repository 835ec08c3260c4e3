/*
 * synth.c -- seeded synthetic inputs and GGUF weight quantizers for the MoE FFN layer.
 *
 * Host-only C (libphxsynth.so).  Used by the tests and bench.py to build the same inputs for the
 * GPU library and the CPU checker.  phoenix-lai itself has no weight-side quantizer (it only
 * quantizes activations), so these encoders are this project's own; any valid block encoding is
 * acceptable because every comparison runs on the decoded arithmetic.
 *
 * Random numbers: each tensor has its own counter-based stream, key = seed ^ FNV-1a-64(name);
 * element i takes the SplitMix64 outputs of counters 2i+1 and 2i+2 as the two uniforms of a
 * Box-Muller pair (double), cast to float.  Deterministic under any thread count.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define GOLDEN 0x9E3779B97F4A7C15ull

static uint64_t mix64(uint64_t z)
{
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

uint64_t phx_synth_key(uint64_t seed, const char* name)
{
    uint64_t h = 0xcbf29ce484222325ull;
    for (const unsigned char* p = (const unsigned char*)name; *p; p++) { h ^= *p; h *= 0x100000001b3ull; }
    return seed ^ h;
}

static double unit(uint64_t key, uint64_t ctr)
{
    /* (0, 1]: never 0, so log() is finite */
    return ((double)(mix64(key + ctr * GOLDEN) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

/* out[i] = mean + std * N(0,1) for element indices offset .. offset+n-1 of the named tensor */
void phx_synth_normal(uint64_t seed, const char* name, float mean, float stdv, float* out, int64_t n, int64_t offset)
{
    const double two_pi = 6.283185307179586476925286766559;
    uint64_t key = phx_synth_key(seed, name);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) {
        uint64_t c = (uint64_t)(offset + i);
        double u1 = unit(key, 2 * c + 1), u2 = unit(key, 2 * c + 2);
        double z = sqrt(-2.0 * log(u1)) * cos(two_pi * u2);
        out[i] = (float)(mean + stdv * z);
    }
}

/* uniform random bytes of the named stream (random block payloads in tests) */
void phx_synth_bytes(uint64_t seed, const char* name, uint8_t* out, int64_t n)
{
    uint64_t key = phx_synth_key(seed, name);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) out[i] = (uint8_t)(mix64(key + (uint64_t)(i + 1) * GOLDEN) >> 56);
}

/* ------------------------------------------------------------------ fp16 (round to nearest even) */

static uint16_t half_from_float(float value)
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

static float half_to_float(uint16_t h)
{
    uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1F, m = h & 0x3FF, bits;
    if (e == 0) {
        if (!m) bits = s;
        else { int k = -1; do { k++; m <<= 1; } while (!(m & 0x400)); bits = s | (uint32_t)(112 - k) << 23 | (m & 0x3FF) << 13; }
    } else if (e == 31) bits = s | 0x7F800000u | m << 13;
    else bits = s | (e + 112) << 23 | m << 13;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static void wr16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* ------------------------------------------------------------------ weight quantizers */

/* Q4_0 (18 B / 32): d = max / -8 over the value of largest |x|, q = min(15, (int)(x/d + 8.5)) */
static void q4_0_block(const float* x, uint8_t* blk)
{
    float amax = 0, max = 0;
    for (int j = 0; j < 32; j++) { float a = fabsf(x[j]); if (a > amax) { amax = a; max = x[j]; } }
    float d = max / -8.0f, id = d != 0 ? 1.0f / d : 0.0f;
    uint16_t dh = half_from_float(d);
    wr16(blk, dh);
    for (int j = 0; j < 16; j++) {
        int q0 = (int)(x[j] * id + 8.5f), q1 = (int)(x[j + 16] * id + 8.5f);
        q0 = q0 < 0 ? 0 : q0 > 15 ? 15 : q0;
        q1 = q1 < 0 ? 0 : q1 > 15 ? 15 : q1;
        blk[2 + j] = (uint8_t)(q0 | (q1 << 4));
    }
}

/* Q8_0 (34 B / 32): d = amax / 127, q = round(x / d) */
static void q8_0_block(const float* x, uint8_t* blk)
{
    float amax = 0;
    for (int j = 0; j < 32; j++) { float a = fabsf(x[j]); if (a > amax) amax = a; }
    float d = amax / 127.0f, id = d != 0 ? 1.0f / d : 0.0f;
    wr16(blk, half_from_float(d));
    for (int j = 0; j < 32; j++) {
        int q = (int)roundf(x[j] * id);
        blk[2 + j] = (uint8_t)(int8_t)(q < -127 ? -127 : q > 127 ? 127 : q);
    }
}

/* Q4_K (144 B / 256): per 32-element sub-block an affine range [lo, hi] with lo <= 0, a 6-bit
 * scale sc and min m under fp16 super-scales d, dmin: value = d*sc*q - dmin*m, q in 0..15. */
static void q4_k_block(const float* x, uint8_t* blk)
{
    float scl[8], mn[8], maxs = 0, maxm = 0;
    for (int s = 0; s < 8; s++) {
        float lo = x[32 * s], hi = x[32 * s];
        for (int j = 1; j < 32; j++) { float v = x[32 * s + j]; if (v < lo) lo = v; if (v > hi) hi = v; }
        if (lo > 0) lo = 0;
        scl[s] = (hi - lo) / 15.0f;
        mn[s] = -lo;
        if (scl[s] > maxs) maxs = scl[s];
        if (mn[s] > maxm) maxm = mn[s];
    }
    uint16_t dh = half_from_float(maxs / 63.0f), mh = half_from_float(maxm / 63.0f);
    float d = half_to_float(dh), dmin = half_to_float(mh);
    int sc[8], m[8];
    for (int s = 0; s < 8; s++) {
        int a = d > 0 ? (int)lrintf(scl[s] / d) : 0, b = dmin > 0 ? (int)lrintf(mn[s] / dmin) : 0;
        sc[s] = a < 0 ? 0 : a > 63 ? 63 : a;
        m[s] = b < 0 ? 0 : b > 63 ? 63 : b;
    }
    wr16(blk, dh);
    wr16(blk + 2, mh);
    uint8_t* q = blk + 4;
    for (int j = 0; j < 4; j++) {
        q[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
        q[j + 4] = (uint8_t)(m[j] | ((m[j + 4] >> 4) << 6));
        q[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
    }
    uint8_t* qs = blk + 16;
    for (int c = 0; c < 4; c++) {
        for (int l = 0; l < 32; l++) {
            int v[2];
            for (int h = 0; h < 2; h++) {
                int s = 2 * c + h;
                float ds = d * sc[s], off = dmin * m[s];
                int qq = ds > 0 ? (int)lrintf((x[32 * s + l] + off) / ds) : 0;
                v[h] = qq < 0 ? 0 : qq > 15 ? 15 : qq;
            }
            qs[32 * c + l] = (uint8_t)(v[0] | (v[1] << 4));
        }
    }
}

/* Q6_K (210 B / 256): per 16-element sub-block a signed int8 scale under an fp16 d:
 * value = d*sc*(q - 32), q in 0..63 (ql: low 4 bits, qh: high 2 bits). */
static void q6_k_block(const float* x, uint8_t* blk)
{
    float scl[16], maxs = 0;
    for (int s = 0; s < 16; s++) {
        float amax = 0, max = 0;
        for (int j = 0; j < 16; j++) { float a = fabsf(x[16 * s + j]); if (a > amax) { amax = a; max = x[16 * s + j]; } }
        scl[s] = max / -32.0f;
        if (fabsf(scl[s]) > maxs) maxs = fabsf(scl[s]);
    }
    uint16_t dh = half_from_float(maxs / 127.0f);
    float d = half_to_float(dh);
    int sc[16];
    for (int s = 0; s < 16; s++) {
        int a = d > 0 ? (int)lrintf(scl[s] / d) : 0;
        sc[s] = a < -128 ? -128 : a > 127 ? 127 : a;
    }
    int q[256];
    for (int e = 0; e < 256; e++) {
        float ds = d * sc[e / 16];
        int v = ds != 0 ? (int)lrintf(x[e] / ds) : 0;
        v = v < -32 ? -32 : v > 31 ? 31 : v;
        q[e] = v + 32;
    }
    uint8_t* ql = blk; uint8_t* qh = blk + 128;
    memset(blk, 0, 210);
    for (int n = 0; n < 2; n++) {
        const int* a = q + 128 * n;
        uint8_t* L = ql + 64 * n; uint8_t* H = qh + 32 * n;
        for (int l = 0; l < 32; l++) {
            L[l] = (uint8_t)((a[l] & 0xF) | ((a[l + 64] & 0xF) << 4));
            L[l + 32] = (uint8_t)((a[l + 32] & 0xF) | ((a[l + 96] & 0xF) << 4));
            H[l] = (uint8_t)((a[l] >> 4) | ((a[l + 32] >> 4) << 2) | ((a[l + 64] >> 4) << 4) | ((a[l + 96] >> 4) << 6));
        }
    }
    for (int s = 0; s < 16; s++) blk[192 + s] = (uint8_t)(int8_t)sc[s];
    wr16(blk + 208, dh);
}

/* Q5_K (176 B / 256): Q4_K's affine sub-blocks with 5-bit q (0..31): d, dmin, the 12 packed scale/min
 * bytes, qh[32] (bit s of qh[l]: the high bit of element 32 s + l), qs[128] (the low nibbles as Q4_K). */
static void q5_k_block(const float* x, uint8_t* blk)
{
    float scl[8], mn[8], maxs = 0, maxm = 0;
    for (int s = 0; s < 8; s++) {
        float lo = x[32 * s], hi = x[32 * s];
        for (int j = 1; j < 32; j++) { float v = x[32 * s + j]; if (v < lo) lo = v; if (v > hi) hi = v; }
        if (lo > 0) lo = 0;
        scl[s] = (hi - lo) / 31.0f;
        mn[s] = -lo;
        if (scl[s] > maxs) maxs = scl[s];
        if (mn[s] > maxm) maxm = mn[s];
    }
    uint16_t dh = half_from_float(maxs / 63.0f), mh = half_from_float(maxm / 63.0f);
    float d = half_to_float(dh), dmin = half_to_float(mh);
    int sc[8], m[8];
    for (int s = 0; s < 8; s++) {
        int a = d > 0 ? (int)lrintf(scl[s] / d) : 0, b = dmin > 0 ? (int)lrintf(mn[s] / dmin) : 0;
        sc[s] = a < 0 ? 0 : a > 63 ? 63 : a;
        m[s] = b < 0 ? 0 : b > 63 ? 63 : b;
    }
    memset(blk, 0, 176);
    wr16(blk, dh);
    wr16(blk + 2, mh);
    uint8_t* q = blk + 4;
    for (int j = 0; j < 4; j++) {
        q[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
        q[j + 4] = (uint8_t)(m[j] | ((m[j + 4] >> 4) << 6));
        q[j + 8] = (uint8_t)((sc[j + 4] & 0xF) | ((m[j + 4] & 0xF) << 4));
    }
    uint8_t* qh = blk + 16;
    uint8_t* qs = blk + 48;
    for (int s = 0; s < 8; s++) {
        float ds = d * sc[s], off = dmin * m[s];
        for (int l = 0; l < 32; l++) {
            int qq = ds > 0 ? (int)lrintf((x[32 * s + l] + off) / ds) : 0;
            qq = qq < 0 ? 0 : qq > 31 ? 31 : qq;
            qs[32 * (s / 2) + l] |= (uint8_t)((qq & 15) << (4 * (s & 1)));
            qh[l] |= (uint8_t)((qq >> 4) << s);
        }
    }
}

/* Q3_K (110 B / 256): per 16-element sub-block a 6-bit signed scale (stored + 32) under an fp16 d:
 * value = d*sc*q, q in -4..3 as q + 4 = (2 low bits in qs) | (hmask bit << 2).  hmask[32] @0, qs[64] @32
 * (element 128 h + 32 j + l: bits 2j of qs[32 h + l]; its hmask bit is bit 4 h + j of hmask[l]),
 * scales[12] @96 (sub-block i: low nibble of byte i (i < 8) or high nibble of byte i - 8, high 2 bits
 * at bits 2 (i / 4) of byte 8 + i % 4), d @108. */
static void q3_k_block(const float* x, uint8_t* blk)
{
    float scl[16], maxs = 0;
    for (int s = 0; s < 16; s++) {
        float amax = 0, max = 0;
        for (int j = 0; j < 16; j++) { float a = fabsf(x[16 * s + j]); if (a > amax) { amax = a; max = x[16 * s + j]; } }
        scl[s] = max / -4.0f;
        if (fabsf(scl[s]) > maxs) maxs = fabsf(scl[s]);
    }
    uint16_t dh = half_from_float(maxs / 31.0f);
    float d = half_to_float(dh);
    int sc[16];
    for (int s = 0; s < 16; s++) {
        int a = d > 0 ? (int)lrintf(scl[s] / d) : 0;
        sc[s] = a < -32 ? -32 : a > 31 ? 31 : a;
    }
    memset(blk, 0, 110);
    uint8_t* hm = blk;
    uint8_t* qs = blk + 32;
    uint8_t* s8 = blk + 96;
    for (int e = 0; e < 256; e++) {
        float ds = d * sc[e / 16];
        int v = ds != 0 ? (int)lrintf(x[e] / ds) : 0;
        v = (v < -4 ? -4 : v > 3 ? 3 : v) + 4;
        int h = e / 128, j = (e % 128) / 32, l = e % 32;
        qs[32 * h + l] |= (uint8_t)((v & 3) << (2 * j));
        hm[l] |= (uint8_t)((v >> 2) << (4 * h + j));
    }
    for (int i = 0; i < 16; i++) {
        int u = sc[i] + 32;
        if (i < 8) s8[i] |= (uint8_t)(u & 15);
        else s8[i - 8] |= (uint8_t)((u & 15) << 4);
        s8[8 + (i % 4)] |= (uint8_t)((u >> 4) << (2 * (i / 4)));
    }
    wr16(blk + 108, dh);
}

int64_t phx_synth_row_bytes(int type, int cols)
{
    switch (type) {
    case 0: return (int64_t)cols * 4;
    case 2: return (int64_t)(cols / 32) * 18;
    case 8: return (int64_t)(cols / 32) * 34;
    case 11: return (int64_t)(cols / 256) * 110;
    case 12: return (int64_t)(cols / 256) * 144;
    case 13: return (int64_t)(cols / 256) * 176;
    case 14: return (int64_t)(cols / 256) * 210;
    }
    return -1;
}

/* rows x cols floats -> rows of GGUF blocks (F32 copies).  Returns 0, or -1/-3 on bad shape/type. */
int phx_synth_quantize(int type, const float* x, int64_t rows, int cols, uint8_t* out)
{
    int64_t rb = phx_synth_row_bytes(type, cols);
    if (rb < 0) return -3;
    int bs = type == 0 ? 1 : (type >= 11 && type <= 14) ? 256 : 32;
    if (cols % bs) return -1;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        const float* xr = x + r * cols;
        uint8_t* o = out + r * rb;
        if (type == 0) { memcpy(o, xr, (size_t)cols * 4); continue; }
        for (int b = 0; b < cols / bs; b++) {
            if (type == 2) q4_0_block(xr + 32 * b, o + 18 * b);
            else if (type == 8) q8_0_block(xr + 32 * b, o + 34 * b);
            else if (type == 11) q3_k_block(xr + 256 * b, o + 110 * b);
            else if (type == 12) q4_k_block(xr + 256 * b, o + 144 * b);
            else if (type == 13) q5_k_block(xr + 256 * b, o + 176 * b);
            else q6_k_block(xr + 256 * b, o + 210 * b);
        }
    }
    return 0;
}

/* Normal rows quantized on the fly, in chunks (no full f32 copy of a large expert tensor).
 * Element (r, c) of the named tensor is counter r*logical_cols + c; columns >= logical_cols (the
 * zero padding of a K-quant row) are 0. */
int phx_synth_quantized_normal(uint64_t seed, const char* name, float mean, float stdv, int type, int64_t rows,
                               int logical_cols, int cols, uint8_t* out)
{
    int64_t rb = phx_synth_row_bytes(type, cols);
    if (rb < 0 || logical_cols > cols) return -1;
    const int64_t chunk = 4096;
    float* buf = (float*)malloc(sizeof(float) * (size_t)chunk * cols);
    if (!buf) return -2;
    for (int64_t r0 = 0; r0 < rows; r0 += chunk) {
        int64_t nr = rows - r0 < chunk ? rows - r0 : chunk;
        if (logical_cols == cols) {
            phx_synth_normal(seed, name, mean, stdv, buf, nr * cols, r0 * cols);
        } else {
            for (int64_t r = 0; r < nr; r++) {
                phx_synth_normal(seed, name, mean, stdv, buf + r * cols, logical_cols, (r0 + r) * logical_cols);
                memset(buf + r * cols + logical_cols, 0, sizeof(float) * (size_t)(cols - logical_cols));
            }
        }
        int rc = phx_synth_quantize(type, buf, nr, cols, out + r0 * rb);
        if (rc) { free(buf); return rc; }
    }
    free(buf);
    return 0;
}

/* ------------------------------------------------------------------ router bias calibration
 * Logits are modelled as N(0, sigma) noise plus a per-expert bias b_e; b is adjusted by
 * fixed-point steps b_e += eta * log(target_e / realised_e) until the top-k selection shares of a
 * seeded Monte Carlo sample match target (normalised to sum k).  Used to bias one input channel of
 * the router (Zipf popularity, or one hot expert). */
void phx_synth_calibrate_bias(uint64_t seed, int E, int k, const double* target, double sigma, int samples,
                              int iters, double* bias)
{
    double* noise = (double*)malloc(sizeof(double) * (size_t)E);
    double* freq = (double*)malloc(sizeof(double) * (size_t)E);
    double* l = (double*)malloc(sizeof(double) * (size_t)E);
    char* taken = (char*)malloc((size_t)E);
    uint64_t key = phx_synth_key(seed, "router.bias.calibration");
    for (int e = 0; e < E; e++) bias[e] = 0;
    for (int it = 0; it < iters; it++) {
        for (int e = 0; e < E; e++) freq[e] = 0;
        for (int s = 0; s < samples; s++) {
            for (int e = 0; e < E; e++) {
                uint64_t c = (uint64_t)s * E + e;
                double z = sqrt(-2.0 * log(unit(key, 2 * c + 1))) * cos(6.283185307179586 * unit(key, 2 * c + 2));
                noise[e] = z;
                l[e] = sigma * z + bias[e];
            }
            memset(taken, 0, (size_t)E);
            for (int j = 0; j < k; j++) {
                int bi = -1;
                for (int e = 0; e < E; e++) if (!taken[e] && (bi < 0 || l[e] > l[bi])) bi = e;
                taken[bi] = 1;
                freq[bi] += 1.0;
            }
        }
        for (int e = 0; e < E; e++) {
            double f = (freq[e] + 0.5) / samples, t = target[e];
            bias[e] += 0.5 * sigma * log(t / f);
        }
    }
    free(noise); free(freq); free(l); free(taken);
}
