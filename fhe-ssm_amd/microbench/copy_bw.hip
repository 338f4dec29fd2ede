// copy_bw.hip -- achievable HBM bandwidth on the GPU it runs on: a grid-stride uint4 copy of a
// 2 GiB buffer (read 2 GiB + write 2 GiB per launch).  Also the reference kernel of known traffic
// against which rocprofv3's FETCH_SIZE / WRITE_SIZE counters are scaled.
// Build: make -C fhe-ssm_amd microbench/copy_bw ; run: fhe-ssm_amd/microbench/copy_bw
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>

__global__ __launch_bounds__(256) void k_copy(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) dst[i] = src[i];
}

int main() {
    const size_t bytes = 2ull << 30, n = bytes / sizeof(uint4);
    uint4 *a = nullptr, *b = nullptr;
    if (hipMalloc(&a, bytes) != hipSuccess || hipMalloc(&b, bytes) != hipSuccess) return 1;
    if (hipMemset(a, 1, bytes) != hipSuccess || hipMemset(b, 0, bytes) != hipSuccess) return 1;
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return 1;
    const int grids[] = {1024, 4096, 16384, 65536};
    for (int gi = 0; gi < 4; gi++) {
        float best = 1e30f;
        for (int rep = 0; rep < 5; rep++) {
            (void)hipEventRecord(e0);
            hipLaunchKernelGGL(k_copy, dim3(grids[gi]), dim3(256), 0, 0, a, b, n);
            (void)hipEventRecord(e1);
            (void)hipEventSynchronize(e1);
            float ms = 0;
            (void)hipEventElapsedTime(&ms, e0, e1);
            if (ms < best) best = ms;
        }
        printf("copy 2 GiB, grid %6d: best %.3f ms  %.1f GB/s (read+write)\n", grids[gi], best,
               2.0 * bytes / (best * 1e-3) / 1e9);
    }
    if (hipDeviceSynchronize() != hipSuccess) return 1;
    (void)hipFree(a);
    (void)hipFree(b);
    return 0;
}
