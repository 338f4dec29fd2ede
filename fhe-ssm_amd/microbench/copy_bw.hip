// copy_bw.hip -- achievable HBM bandwidth on the GPU it runs on, and the reference kernels of known traffic against
// which rocprofv3's FETCH_SIZE / WRITE_SIZE counters are scaled.
//
// Kernels (every byte of the buffers touched exactly once per launch; sizes well above the 256 MiB memory-side cache):
//   k_copy        the counter reference: a grid-stride uint4 copy of 2 GiB (read 2 GiB + write 2 GiB)
//   k_read<U>     read-only stream: U 16-byte nontemporal loads in flight per thread, folded with XOR into one word per
//                 thread (the only write: grid x 8 B)
//   k_copy_u<U,NT> copy stream: U 16-byte loads in flight per thread, then their U stores; NT = nontemporal loads and
//                 stores (the engine's hint for data a kernel touches once), else ordinary ones
//   k_write<U>    write-only stream: U 16-byte nontemporal stores per thread per iteration
// Each thread of a stream kernel walks the buffer in steps of grid x 256 x U uint4, its U accesses 256 uint4 apart
// (so every load instruction of a wave reads 1 KiB of consecutive bytes).
// Build: make -C fhe-ssm_amd microbench/copy_bw ; run: fhe-ssm_amd/microbench/copy_bw [--quick]
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
#include <cstring>

#define HIPCK(x)                                                                        \
    do {                                                                                \
        hipError_t e_ = (x);                                                            \
        if (e_ != hipSuccess) {                                                         \
            fprintf(stderr, "%s:%d %s: %s\n", __FILE__, __LINE__, #x, hipGetErrorString(e_)); \
            return 1;                                                                   \
        }                                                                               \
    } while (0)

// a native 16-byte vector (the nontemporal builtins take vector types, not HIP's uint4 struct)
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void k_copy(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) dst[i] = src[i];
}

// n: 16-byte word count, a multiple of gridDim.x * 256 * U (checked on the host)
template <int U>
__global__ __launch_bounds__(256) void k_read(const v4u* __restrict__ src, uint64_t* __restrict__ sink, size_t n) {
    const size_t stride = (size_t)gridDim.x * 256 * U;
    uint32_t acc = 0;
    for (size_t base = (size_t)blockIdx.x * 256 * U + threadIdx.x; base < n; base += stride) {
        v4u v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = __builtin_nontemporal_load(&src[base + (size_t)u * 256]);
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    sink[(size_t)blockIdx.x * 256 + threadIdx.x] = acc;
}

template <int U, bool NT>
__global__ __launch_bounds__(256) void k_copy_u(const v4u* __restrict__ src, v4u* __restrict__ dst, size_t n) {
    const size_t stride = (size_t)gridDim.x * 256 * U;
    for (size_t base = (size_t)blockIdx.x * 256 * U + threadIdx.x; base < n; base += stride) {
        v4u v[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (NT)
                v[u] = __builtin_nontemporal_load(&src[base + (size_t)u * 256]);
            else
                v[u] = src[base + (size_t)u * 256];
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (NT)
                __builtin_nontemporal_store(v[u], &dst[base + (size_t)u * 256]);
            else
                dst[base + (size_t)u * 256] = v[u];
        }
    }
}

template <int U>
__global__ __launch_bounds__(256) void k_write(v4u* __restrict__ dst, size_t n, uint32_t val) {
    const size_t stride = (size_t)gridDim.x * 256 * U;
    const v4u v = {val, val ^ 1u, val ^ 2u, val ^ 3u};
    for (size_t base = (size_t)blockIdx.x * 256 * U + threadIdx.x; base < n; base += stride) {
#pragma unroll
        for (int u = 0; u < U; u++) __builtin_nontemporal_store(v, &dst[base + (size_t)u * 256]);
    }
}

struct Timer {
    hipEvent_t e0, e1;
};

template <typename F>
static float best_ms(Timer& t, int reps, F launch) {
    float best = 1e30f;
    for (int r = 0; r < reps; r++) {
        (void)hipEventRecord(t.e0);
        launch();
        (void)hipEventRecord(t.e1);
        (void)hipEventSynchronize(t.e1);
        float ms = 0;
        (void)hipEventElapsedTime(&ms, t.e0, t.e1);
        if (ms < best) best = ms;
    }
    return best;
}

template <int U>
static int sweep(Timer& t, const v4u* a, v4u* b, uint64_t* sink, size_t bytes, const int* grids, int ng, int reps) {
    const size_t n = bytes / sizeof(v4u);
    for (int gi = 0; gi < ng; gi++) {
        const int g = grids[gi];
        if (n % ((size_t)g * 256 * U)) continue;
        float r = best_ms(t, reps, [&] { hipLaunchKernelGGL((k_read<U>), dim3(g), dim3(256), 0, 0, a, sink, n); });
        HIPCK(hipGetLastError());
        float cn = best_ms(t, reps, [&] { hipLaunchKernelGGL((k_copy_u<U, true>), dim3(g), dim3(256), 0, 0, a, b, n); });
        HIPCK(hipGetLastError());
        float cp = best_ms(t, reps, [&] { hipLaunchKernelGGL((k_copy_u<U, false>), dim3(g), dim3(256), 0, 0, a, b, n); });
        HIPCK(hipGetLastError());
        float w = best_ms(t, reps, [&] { hipLaunchKernelGGL((k_write<U>), dim3(g), dim3(256), 0, 0, b, n, 7u); });
        HIPCK(hipGetLastError());
        printf("| %5.1f | %2d | %6d | %8.1f | %8.1f | %8.1f | %8.1f |\n", bytes / 1073741824.0, U, g,
               bytes / (r * 1e-3) / 1e9, 2.0 * bytes / (cn * 1e-3) / 1e9, 2.0 * bytes / (cp * 1e-3) / 1e9,
               bytes / (w * 1e-3) / 1e9);
        fflush(stdout);
    }
    return 0;
}

int main(int argc, char** argv) {
    const bool quick = argc > 1 && !strcmp(argv[1], "--quick");
    // the counter reference: 2 GiB copy, grid 16384 (the figure the counter scaling in profiles/ reads)
    const size_t ref_bytes = 2ull << 30;
    const size_t max_bytes = quick ? (4ull << 30) : (8ull << 30);
    uint4 *a = nullptr, *b = nullptr;
    uint64_t* sink = nullptr;
    HIPCK(hipMalloc(&a, max_bytes));
    HIPCK(hipMalloc(&b, max_bytes));
    HIPCK(hipMalloc(&sink, (size_t)65536 * 256 * 8));
    HIPCK(hipMemset(a, 1, max_bytes));
    HIPCK(hipMemset(b, 0, max_bytes));
    Timer t;
    HIPCK(hipEventCreate(&t.e0));
    HIPCK(hipEventCreate(&t.e1));
    {
        const size_t n = ref_bytes / sizeof(uint4);
        float ms = best_ms(t, 5, [&] { hipLaunchKernelGGL(k_copy, dim3(16384), dim3(256), 0, 0, a, b, n); });
        HIPCK(hipGetLastError());
        printf("reference copy (k_copy) 2 GiB, grid 16384: best %.3f ms, %.1f GB/s (read + write)\n\n", ms,
               2.0 * ref_bytes / (ms * 1e-3) / 1e9);
    }
    printf("| GiB per buffer | loads in flight U | grid | read GB/s | copy NT GB/s | copy GB/s | write NT GB/s |\n");
    printf("|---|---|---|---|---|---|---|\n");
    const int grids[] = {1024, 2048, 4096, 8192, 16384};
    const int reps = quick ? 3 : 5;
    for (size_t bytes = 4ull << 30; bytes <= max_bytes; bytes <<= 1) {
        if (sweep<1>(t, (const v4u*)a, (v4u*)b, sink, bytes, grids, 5, reps)) return 1;
        if (sweep<2>(t, (const v4u*)a, (v4u*)b, sink, bytes, grids, 5, reps)) return 1;
        if (sweep<4>(t, (const v4u*)a, (v4u*)b, sink, bytes, grids, 5, reps)) return 1;
        if (sweep<8>(t, (const v4u*)a, (v4u*)b, sink, bytes, grids, 5, reps)) return 1;
    }
    HIPCK(hipDeviceSynchronize());
    (void)hipFree(a);
    (void)hipFree(b);
    (void)hipFree(sink);
    return 0;
}
