// mall_bw.hip -- can data one kernel writes be read back by the next from the memory-side Infinity Cache (MALL,
// 256 MiB on MI355X) faster than from HBM?  For working sets S from 8 MiB to 1 GiB:
//   read   repeated read-only sweeps of S (a reduction into one word per workgroup), GB/s of the second sweep;
//   w->r   a kernel writes S (ordinary stores), the next kernel reads S: GB/s of the read kernel;
//   w->r nt  the same with nontemporal stores.
// The NTT's two-pass schedule writes every limb between its passes; if written data stays in the MALL at a
// working set of a few hundred limbs, chunking the passes could take that round trip off HBM.
// Build: make -C fhe-ssm_amd microbench/mall_bw ; run: fhe-ssm_amd/microbench/mall_bw
#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstdio>

__global__ __launch_bounds__(256) void k_read(const uint4* __restrict__ src, size_t n, uint32_t* __restrict__ out) {
    uint32_t acc = 0;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const uint4 v = src[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9e3779b9u) out[blockIdx.x] = acc;  // keeps the loads; never true for the fill pattern
}

template <bool NT>
__global__ __launch_bounds__(256) void k_write(uint4* __restrict__ dst, size_t n, uint32_t salt) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const uint4 v = make_uint4((uint32_t)i, salt, (uint32_t)i ^ salt, 1u);
        if (NT) {
            uint32_t* d = reinterpret_cast<uint32_t*>(&dst[i]);
            __builtin_nontemporal_store(v.x, d);
            __builtin_nontemporal_store(v.y, d + 1);
            __builtin_nontemporal_store(v.z, d + 2);
            __builtin_nontemporal_store(v.w, d + 3);
        } else {
            dst[i] = v;
        }
    }
}

int main() {
    const size_t max_bytes = 1ull << 30;
    uint4* buf = nullptr;
    uint32_t* out = nullptr;
    if (hipMalloc(&buf, max_bytes) != hipSuccess || hipMalloc(&out, 65536 * 4) != hipSuccess) return 1;
    if (hipMemset(buf, 1, max_bytes) != hipSuccess) return 1;
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return 1;
    const int grid = 8192;
    auto timed = [&](auto launch) {
        float best = 1e30f;
        for (int rep = 0; rep < 5; rep++) {
            (void)hipEventRecord(e0);
            launch();
            (void)hipEventRecord(e1);
            (void)hipEventSynchronize(e1);
            float ms = 0;
            (void)hipEventElapsedTime(&ms, e0, e1);
            if (ms < best) best = ms;
        }
        return best;
    };
    printf("%10s %12s %12s %12s\n", "MiB", "read GB/s", "w->r GB/s", "w(nt)->r GB/s");
    for (size_t mib = 8; mib <= 1024; mib *= 2) {
        const size_t bytes = mib << 20, n = bytes / sizeof(uint4);
        // read: one warming sweep, then the timed sweeps (best of 5)
        hipLaunchKernelGGL(k_read, dim3(grid), dim3(256), 0, 0, buf, n, out);
        const float t_read = timed([&] { hipLaunchKernelGGL(k_read, dim3(grid), dim3(256), 0, 0, buf, n, out); });
        // write then read: only the read kernel is timed
        float t_wr = 1e30f, t_wr_nt = 1e30f;
        for (int rep = 0; rep < 5; rep++) {
            hipLaunchKernelGGL(k_write<false>, dim3(grid), dim3(256), 0, 0, buf, n, (uint32_t)rep);
            (void)hipEventRecord(e0);
            hipLaunchKernelGGL(k_write<false>, dim3(grid), dim3(256), 0, 0, buf, n, (uint32_t)rep + 7);
            (void)hipEventRecord(e1);
            (void)hipEventSynchronize(e1);
            (void)hipEventRecord(e0);
            hipLaunchKernelGGL(k_read, dim3(grid), dim3(256), 0, 0, buf, n, out);
            (void)hipEventRecord(e1);
            (void)hipEventSynchronize(e1);
            float ms = 0;
            (void)hipEventElapsedTime(&ms, e0, e1);
            if (ms < t_wr) t_wr = ms;
            hipLaunchKernelGGL(k_write<true>, dim3(grid), dim3(256), 0, 0, buf, n, (uint32_t)rep + 13);
            (void)hipEventRecord(e0);
            hipLaunchKernelGGL(k_read, dim3(grid), dim3(256), 0, 0, buf, n, out);
            (void)hipEventRecord(e1);
            (void)hipEventSynchronize(e1);
            ms = 0;
            (void)hipEventElapsedTime(&ms, e0, e1);
            if (ms < t_wr_nt) t_wr_nt = ms;
        }
        printf("%10zu %12.1f %12.1f %12.1f\n", mib, bytes / (t_read * 1e-3) / 1e9, bytes / (t_wr * 1e-3) / 1e9,
               bytes / (t_wr_nt * 1e-3) / 1e9);
        fflush(stdout);
    }
    if (hipDeviceSynchronize() != hipSuccess) return 1;
    (void)hipFree(buf);
    (void)hipFree(out);
    return 0;
}
