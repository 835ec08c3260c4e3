// MI355X probe: the gap between dependent kernels in a replayed HIP graph (last workgroup's end to the
// next kernel's first start, from wall-clock stamps) for grids of 128-512 workgroups, 256 or 1024
// threads, 1 KB or 64 KB of LDS, 24-byte or 1-KB kernel arguments, with and without stores.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <vector>
#include <algorithm>
#define CK(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { printf("HIP error %s at %d\n", hipGetErrorString(e_), __LINE__); exit(1);} } while (0)

struct Big { unsigned long long* st; float* out; int idx, nwrite; char pad[1000]; };
struct Small { unsigned long long* st; float* out; int idx, nwrite; };

template <class A>
__global__ void k_stamp(A a)
{
    extern __shared__ float lds[];
    const unsigned long long t0 = wall_clock64();
    // a little work
    if (a.nwrite) for (int i = threadIdx.x; i < a.nwrite; i += blockDim.x) a.out[(long)blockIdx.x * a.nwrite + i] = (float)i;
    lds[threadIdx.x] = 1.0f;
    __syncthreads();
    if (threadIdx.x == 0) {
        a.st[(a.idx * 1024 + blockIdx.x) * 2] = t0;
        a.st[(a.idx * 1024 + blockIdx.x) * 2 + 1] = wall_clock64();
    }
}

int main()
{
    unsigned long long* st; float* out;
    CK(hipMalloc(&st, 64 * 1024 * 2 * 8));
    CK(hipMalloc(&out, 64L << 20));
    hipStream_t s; CK(hipStreamCreate(&s));
    std::vector<unsigned long long> h(64 * 1024 * 2);
    const int NK = 20;
    for (int big = 0; big < 2; big++)
    for (int grid : {128, 256, 512})
    for (int block : {256, 1024})
    for (int lds : {1024, 65536})
    for (int nwrite : {0, 1024}) {
        if (lds > 65536) continue;
        if (big) CK(hipFuncSetAttribute((const void*)k_stamp<Big>, hipFuncAttributeMaxDynamicSharedMemorySize, 65536));
        else CK(hipFuncSetAttribute((const void*)k_stamp<Small>, hipFuncAttributeMaxDynamicSharedMemorySize, 65536));
        hipGraph_t g; hipGraphExec_t ge;
        CK(hipStreamBeginCapture(s, hipStreamCaptureModeGlobal));
        for (int i = 0; i < NK; i++) {
            if (big) { Big a{}; a.st = st; a.out = out; a.idx = i; a.nwrite = nwrite; hipLaunchKernelGGL(k_stamp<Big>, dim3(grid), dim3(block), lds, s, a); }
            else { Small a{st, out, i, nwrite}; hipLaunchKernelGGL(k_stamp<Small>, dim3(grid), dim3(block), lds, s, a); }
        }
        CK(hipStreamEndCapture(s, &g));
        CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        for (int r = 0; r < 5; r++) CK(hipGraphLaunch(ge, s));
        CK(hipStreamSynchronize(s));
        CK(hipMemcpy(h.data(), st, h.size() * 8, hipMemcpyDeviceToHost));
        double gap = 0, dur = 0; int n = 0;
        for (int i = 1; i < NK - 1; i++) {
            unsigned long long e0 = 0, s1 = ~0ull, s0 = ~0ull;
            for (int b = 0; b < grid; b++) { e0 = std::max(e0, h[((i - 1) * 1024 + b) * 2 + 1]); s1 = std::min(s1, h[(i * 1024 + b) * 2]); s0 = std::min(s0, h[((i-1) * 1024 + b) * 2]); }
            gap += ((double)s1 - (double)e0) / 100.0; dur += ((double)e0 - (double)s0) / 100.0; n++;
        }
        printf("kernarg %-5s grid %4d block %4d lds %6d write/WG %5d floats: gap %.2f us, kernel span %.2f us\n", big ? "1KB" : "24B", grid, block, lds, nwrite, gap / n, dur / n);
        CK(hipGraphExecDestroy(ge)); CK(hipGraphDestroy(g));
    }
    return 0;
}
