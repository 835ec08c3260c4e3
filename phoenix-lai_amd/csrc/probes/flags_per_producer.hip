// MI355X probe: one flag word per producer.  P producer workgroups write 256 B and release-store their
// own word at agent scope (mode 0: a release store; mode 1: a release fence, then a relaxed store); the
// other workgroups poll all P words with relaxed agent-scope loads, acquire, then read the data.  Polls
// are bounded (no wait outlives its limit).
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <vector>
#include <algorithm>
#define CK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { printf("HIP error %s at %d\n", hipGetErrorString(e_), __LINE__); exit(1);} } while (0)

__global__ __launch_bounds__(256) void k_flags(int P, unsigned* flags, unsigned epoch, float* data, unsigned long long* st, int* err, int spin_max, int mode)
{
    const int wg = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const unsigned long long t0 = wall_clock64();
    // every WG does ~1 us of "work" first (spin on the clock) so consumers are already polling
    if (wg < P) {
        while (wall_clock64() - t0 < 200) {}
        if (tid < 64) data[wg * 64 + tid] = (float)(wg * 1000 + tid) + (float)epoch;
        __syncthreads();
        if (tid == 0) {
            const unsigned long long tr0 = wall_clock64();
            if (mode == 0) __hip_atomic_store(&flags[wg * 16], epoch, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            else { __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent"); __hip_atomic_store(&flags[wg * 16], epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
            st[wg * 4 + 0] = t0; st[wg * 4 + 1] = tr0; st[wg * 4 + 2] = wall_clock64(); st[wg * 4 + 3] = 0;
        }
    } else {
        __shared__ float red[4];
        if (tid < 64) {
            int it = 0; bool all = false;
            while (!all && it < spin_max) {
                bool mine = true;
                for (int p = lane; p < P; p += 64) mine &= __hip_atomic_load(&flags[p * 16], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == epoch;
                all = __all(mine);
                it++;
            }
            if (!all && lane == 0) atomicAdd(err, 1);
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            if (lane == 0) { st[wg * 4 + 0] = t0; st[wg * 4 + 1] = wall_clock64(); }
        }
        __syncthreads();
        float s = 0.0f;
        for (int p = tid >> 6; p < P; p += 4) s += data[p * 64 + lane];
        for (int m = 32; m; m >>= 1) s += __shfl_xor(s, m, 64);
        if (lane == 0) red[tid >> 6] = s;
        __syncthreads();
        if (tid == 0) { st[wg * 4 + 2] = wall_clock64(); st[wg * 4 + 3] = (unsigned long long)__float_as_uint(red[0] + red[1] + red[2] + red[3]); }
    }
}

int main()
{
    const int NWG = 256;
    unsigned* flags; int* err; float* data; unsigned long long* st;
    CK(hipMalloc(&flags, NWG * 64)); CK(hipMemset(flags, 0, NWG * 64));
    CK(hipMalloc(&err, 4)); CK(hipMalloc(&data, NWG * 64 * 4)); CK(hipMalloc(&st, NWG * 32));
    std::vector<unsigned long long> h(NWG * 4);
    unsigned epoch = 1;
    for (int mode = 0; mode < 2; mode++)
    for (int P : {8, 22, 64, 128, 176}) {
        for (int rep = 0; rep < 3; rep++, epoch++) {
            CK(hipMemset(err, 0, 4));
            hipLaunchKernelGGL(k_flags, dim3(NWG), dim3(256), 0, 0, P, flags, epoch, data, st, err, 100000, mode);
            CK(hipDeviceSynchronize());
            int e; CK(hipMemcpy(&e, err, 4, hipMemcpyDeviceToHost));
            CK(hipMemcpy(h.data(), st, NWG * 32, hipMemcpyDeviceToHost));
            unsigned long long lastrel = 0, firstrel = ~0ull, relc = 0, smin = ~0ull, smax = 0, rmax = 0;
            for (int i = 0; i < P; i++) { lastrel = std::max(lastrel, h[i*4+2]); firstrel = std::min(firstrel, h[i*4+1]); relc = std::max(relc, h[i*4+2]-h[i*4+1]); }
            for (int i = P; i < NWG; i++) { smin = std::min(smin, h[i*4+1]); smax = std::max(smax, h[i*4+1]); rmax = std::max(rmax, h[i*4+2]-h[i*4+1]); }
            printf("mode %d P=%3d rep %d err=%d: releases span %.2f us (max one %.2f), flags all seen %.2f..%.2f us after the last release, data read after %.2f us\n",
                   mode, P, rep, e, (lastrel - firstrel) / 100.0, relc / 100.0, ((double)smin - lastrel) / 100.0, ((double)smax - lastrel) / 100.0, rmax / 100.0);
        }
    }
    return 0;
}
