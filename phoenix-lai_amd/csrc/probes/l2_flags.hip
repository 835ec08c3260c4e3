// MI355X probes: (1) one shared counter: P producer workgroups write 64 KB each and increment one
// counter with release semantics at agent scope, the other workgroups poll it and then read a producer's
// data; (2) L2 across launches: a launch of 256 workgroups rereads 12 or 48 MB that the previous launch
// read, with workgroup b reading what workgroup b, b + 1 or b + 8 read (workgroup b of a launch runs on
// XCD b % 8), against a cold read after a 1 GB flush.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <vector>
#include <algorithm>
#define CK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { printf("HIP error %s at %d\n", hipGetErrorString(e_), __LINE__); exit(1);} } while (0)

__global__ __launch_bounds__(256) void k_flag(int P, int* cnt, float4* data, int slice4, unsigned long long* st, int* err, int spin_max, int mode)
{
    const int wg = blockIdx.x, tid = threadIdx.x;
    const unsigned long long t0 = wall_clock64();
    if (wg < P) {
        float4 v = make_float4((float)wg, (float)tid, 1.0f, 2.0f);
        for (int i = tid; i < slice4; i += blockDim.x) data[(long)wg * slice4 + i] = v;
        __syncthreads();
        if (tid == 0) {
            const unsigned long long tr0 = wall_clock64();
            if (mode == 0) __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            else {
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
                __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            const unsigned long long tr1 = wall_clock64();
            st[wg * 4 + 0] = t0; st[wg * 4 + 1] = tr0; st[wg * 4 + 2] = tr1; st[wg * 4 + 3] = 0;
        }
    } else {
        __shared__ float red[4];
        if (tid == 0) {
            int n = 0, it = 0;
            while ((n = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) < P && it < spin_max) {
                it++;
                __builtin_amdgcn_s_sleep(1);
            }
            if (n < P) atomicAdd(err, 1);
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            st[wg * 4 + 0] = t0;
            st[wg * 4 + 1] = wall_clock64();
        }
        __syncthreads();
        const int src = (wg * 3 + 1) % P;
        float s = 0.0f;
        for (int i = tid; i < slice4; i += blockDim.x) s += data[(long)src * slice4 + i].x;
        for (int m = 32; m; m >>= 1) s += __shfl_xor(s, m, 64);
        if ((tid & 63) == 0) red[tid >> 6] = s;
        __syncthreads();
        if (tid == 0) {
            st[wg * 4 + 2] = wall_clock64();
            st[wg * 4 + 3] = (unsigned long long)__float_as_uint(red[0] + red[1] + red[2] + red[3]);
        }
    }
}

// WG i reads slice (i + shift) % n: 16-byte loads, all issued then summed
__global__ __launch_bounds__(256) void k_read(const float4* buf, int slice4, int shift, float* sink, unsigned long long* st)
{
    const int wg = blockIdx.x, tid = threadIdx.x, n = gridDim.x;
    const unsigned long long t0 = wall_clock64();
    const float4* p = buf + (long)((wg + shift) % n) * slice4;
    float s = 0.0f;
    for (int i = tid; i < slice4; i += 256) { float4 v = p[i]; s += v.x + v.y + v.z + v.w; }
    for (int m = 32; m; m >>= 1) s += __shfl_xor(s, m, 64);
    if ((tid & 63) == 0) atomicAdd(sink, s);
    __syncthreads();
    if (tid == 0) { st[wg * 2] = t0; st[wg * 2 + 1] = wall_clock64(); }
}

__global__ void k_flush(const float4* buf, long n4, float* sink)
{
    float s = 0.0f;
    for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += (long)gridDim.x * blockDim.x) s += buf[i].x;
    if (s == 12345.0f) *sink = s;
}

int main()
{
    int clk_khz = 0;
    CK(hipDeviceGetAttribute(&clk_khz, hipDeviceAttributeWallClockRate, 0));
    const double us_per_tick = 1000.0 / clk_khz;
    printf("wall clock %d kHz\n", clk_khz);
    const int NWG = 256;
    int *cnt, *err; float4* data; unsigned long long* st; float* sink;
    CK(hipMalloc(&cnt, 4)); CK(hipMalloc(&err, 4)); CK(hipMalloc(&sink, 4));
    CK(hipMalloc(&st, NWG * 4 * 8));
    const long flushB = 1L << 30;
    float4* flush; CK(hipMalloc(&flush, flushB)); CK(hipMemset(flush, 0, flushB));
    std::vector<unsigned long long> h(NWG * 4);
    // ---- flag latency
    for (int mode = 0; mode < 2; mode++)
    for (int P : {8, 64, 176}) {
        const int slice4 = 64 * 1024 / 16;  // 64 KB per producer
        CK(hipMalloc(&data, (long)P * slice4 * 16));
        for (int rep = 0; rep < 3; rep++) {
            CK(hipMemset(cnt, 0, 4)); CK(hipMemset(err, 0, 4));
            hipLaunchKernelGGL(k_flag, dim3(NWG), dim3(256), 0, 0, P, cnt, data, slice4, st, err, 2000000, mode);
            CK(hipDeviceSynchronize());
            int e; CK(hipMemcpy(&e, err, 4, hipMemcpyDeviceToHost));
            CK(hipMemcpy(h.data(), st, NWG * 4 * 8, hipMemcpyDeviceToHost));
            unsigned long long tmin = ~0ull, lastrel = 0, rel_cost = 0, seen_min = ~0ull, seen_max = 0, read_max = 0, read_sum = 0;
            for (int i = 0; i < NWG; i++) tmin = std::min(tmin, h[i * 4]);
            for (int i = 0; i < P; i++) { lastrel = std::max(lastrel, h[i * 4 + 2]); rel_cost = std::max(rel_cost, h[i * 4 + 2] - h[i * 4 + 1]); }
            for (int i = P; i < NWG; i++) {
                seen_min = std::min(seen_min, h[i * 4 + 1]); seen_max = std::max(seen_max, h[i * 4 + 1]);
                read_max = std::max(read_max, h[i * 4 + 2] - h[i * 4 + 1]); read_sum += h[i * 4 + 2] - h[i * 4 + 1];
            }
            printf("flag mode %d P=%3d rep %d err=%d: last release done %.2f us, max release cost %.2f us, consumers see flag %.2f..%.2f us after last release, cold 64KB read max %.2f avg %.2f us\n",
                   mode, P, rep, e, (lastrel - tmin) * us_per_tick, rel_cost * us_per_tick, ((double)seen_min - (double)lastrel) * us_per_tick,
                   ((double)seen_max - (double)lastrel) * us_per_tick, read_max * us_per_tick, read_sum * us_per_tick / (NWG - P));
        }
        CK(hipFree(data));
    }
    // ---- retention across kernel boundaries
    for (long total : {12L << 20, 48L << 20}) {
        const int slice4 = (int)(total / NWG / 16);
        float4 *A, *B; CK(hipMalloc(&A, total)); CK(hipMalloc(&B, total));
        CK(hipMemset(A, 0, total)); CK(hipMemset(B, 0, total));
        hipEvent_t e0, e1; CK(hipEventCreate(&e0)); CK(hipEventCreate(&e1));
        auto run = [&](const char* name, const float4* buf, int shift, bool flush_first) {
            if (flush_first) hipLaunchKernelGGL(k_flush, dim3(4096), dim3(256), 0, 0, flush, flushB / 16, sink);
            CK(hipEventRecord(e0, 0));
            hipLaunchKernelGGL(k_read, dim3(NWG), dim3(256), 0, 0, buf, slice4, shift, sink, st);
            CK(hipEventRecord(e1, 0));
            CK(hipDeviceSynchronize());
            float ms; CK(hipEventElapsedTime(&ms, e0, e1));
            CK(hipMemcpy(h.data(), st, NWG * 2 * 8, hipMemcpyDeviceToHost));
            unsigned long long a = ~0ull, b = 0, mx = 0;
            for (int i = 0; i < NWG; i++) { a = std::min(a, h[i * 2]); b = std::max(b, h[i * 2 + 1]); mx = std::max(mx, h[i*2+1]-h[i*2]); }
            printf("  %-40s total %5.1f MB: event %.2f us, stamps span %.2f us, max WG %.2f us\n", name, total / 1048576.0, ms * 1000.0,
                   (b - a) * us_per_tick, mx * us_per_tick);
        };
        for (int rep = 0; rep < 2; rep++) {
            run("cold (after 1 GB flush)", A, 0, true);
            run("same mapping again", A, 0, false);
            run("shifted by 1 WG (other XCD)", A, 1, false);
            run("shifted by 8 WGs (same XCD?)", A, 8, false);
            run("other buffer, not flushed (cold?)", B, 0, false);
        }
        CK(hipFree(A)); CK(hipFree(B));
    }
    printf("done\n");
    return 0;
}
