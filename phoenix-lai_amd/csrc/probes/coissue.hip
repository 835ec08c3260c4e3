// MI355X probe: do MFMA and VALU instructions of different waves overlap on one SIMD?  One workgroup
// per CU of 8, 12 or 16 waves; waves 0-3 (one per SIMD: a workgroup's wave w runs on SIMD w % 4) loop
// on four independent v_mfma_f32_32x32x16_f16, the others on 16 independent multiply-add chains (32
// VALU instructions per iteration, no FMA contraction: built with -ffp-contract=off).  Mode 1 runs the
// MFMA waves alone, mode 2 the VALU waves alone, mode 3 both; each wave stamps the 100 MHz wall clock
// around its loop and the program prints cycles per iteration at 2.4 GHz.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#define CK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { printf("HIP error %s at %d\n", hipGetErrorString(e_), __LINE__); exit(1);} } while (0)
typedef _Float16 mh8 __attribute__((ext_vector_type(8)));
typedef float mf16 __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(1024) void k_ovl(int mode, int iters, float* out, unsigned long long* st)
{
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const unsigned long long t0 = wall_clock64();
    float res = 0.0f;
    if (wave < 4 && (mode & 1)) {
        mh8 a, b;
        for (int i = 0; i < 8; i++) { a[i] = (_Float16)(lane + i); b[i] = (_Float16)(i - lane); }
        mf16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
        for (int it = 0; it < iters; it++) {
            c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c3, 0, 0, 0);
        }
        for (int q = 0; q < 16; q++) res += c0[q] + c1[q] + c2[q] + c3[q];
    }
    if (wave >= 4 && (mode & 2)) {
        float s[16], x[16];
        for (int q = 0; q < 16; q++) { s[q] = lane * 0.1f + q; x[q] = 1.0f + q * 1e-3f; }
        for (int it = 0; it < iters; it++) {
            // 32 VALU: 16 independent mul+add chains (like the block chain)
#pragma unroll
            for (int q = 0; q < 16; q++) s[q] = s[q] + x[q] * s[(q + 1) & 15];
            asm volatile("" : "+v"(s[0]), "+v"(s[1]), "+v"(s[2]), "+v"(s[3]), "+v"(s[4]), "+v"(s[5]), "+v"(s[6]), "+v"(s[7]));
        }
        for (int q = 0; q < 16; q++) res += s[q];
    }
    const unsigned long long t1 = wall_clock64();
    out[blockIdx.x * 1024 + threadIdx.x] = res;
    if (lane == 0) { st[(blockIdx.x * 16 + wave) * 2] = t0; st[(blockIdx.x * 16 + wave) * 2 + 1] = t1; }
}

int main()
{
    float* out; unsigned long long* st;
    const int NB = 256;
    CK(hipMalloc(&out, NB * 1024 * 4)); CK(hipMalloc(&st, NB * 16 * 16));
    static unsigned long long h[NB * 32];
    const int iters = 4000;
    for (int nw : {8, 12, 16})
    for (int mode = 1; mode <= 3; mode++) {
        hipLaunchKernelGGL(k_ovl, dim3(NB), dim3(nw * 64), 0, 0, mode, iters, out, st);
        CK(hipDeviceSynchronize());
        CK(hipMemcpy(h, st, sizeof(h), hipMemcpyDeviceToHost));
        double mf = 0, va = 0;
        for (int b = 0; b < NB; b++) for (int w = 0; w < nw; w++) {
            double d = (h[(b * 16 + w) * 2 + 1] - h[(b * 16 + w) * 2]) / 100.0;
            if (w < 4) mf = std::max(mf, d); else va = std::max(va, d);
        }
        // cycles per iteration at 2.4 GHz
        printf("waves %d (VALU waves per SIMD %d) mode %d: mfma waves %.1f us (%.1f cyc/iter of 4 MFMA), valu waves %.1f us (%.1f cyc/iter of 32 VALU)\n", nw, nw / 4 - 1, mode,
               mf, mf * 2400.0 / iters, va, va * 2400.0 / iters);
    }
    return 0;
}
