// valu_rate.hip -- issue rate of the VALU instructions the 64-bit modular arithmetic is built from
// (v_mad_u64_u32, v_mul_lo/hi_u32, 24-bit multiplies, v_fma_f64, adds) on the GPU it runs on.  Each thread
// runs 8 independent dependency chains of one instruction; the figure printed is cycles per wave64
// instruction per SIMD (4.0 = one 16-lane pass per cycle for 4 cycles: full rate).
// Build: make -C fhe-ssm_amd microbench/valu_rate ; run: fhe-ssm_amd/microbench/valu_rate
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdint>
#define ITERS 512
template <int OP>
__global__ __launch_bounds__(256) void kern(uint64_t* out, uint32_t seed) {
  uint64_t a0 = threadIdx.x + seed, a1 = a0 * 3, a2 = a0 * 5, a3 = a0 * 7, a4 = a0*11, a5=a0*13, a6=a0*17, a7=a0*19;
  uint32_t b = seed | 1, c = seed ^ 0x1234567;
  double d0 = a0, d1 = a1, d2 = a2, d3 = a3, d4=a4, d5=a5, d6=a6, d7=a7; double e = 1.0000001, f = 0.999;
  uint32_t u0 = a0, u1 = a1, u2 = a2, u3 = a3, u4=a4,u5=a5,u6=a6,u7=a7;
  for (int i = 0; i < ITERS; i++) {
    if (OP == 0) {  // v_mad_u64_u32
#define M(x) asm volatile("v_mad_u64_u32 %0, vcc, %1, %2, %0" : "+v"(x) : "v"(b), "v"(c) : "vcc");
      M(a0) M(a1) M(a2) M(a3) M(a4) M(a5) M(a6) M(a7)
    } else if (OP == 1) {  // v_mul_lo_u32
#define ML(x) asm volatile("v_mul_lo_u32 %0, %0, %1" : "+v"(x) : "v"(b));
      ML(u0) ML(u1) ML(u2) ML(u3) ML(u4) ML(u5) ML(u6) ML(u7)
    } else if (OP == 2) {  // v_mul_hi_u32
#define MH(x) asm volatile("v_mul_hi_u32 %0, %0, %1" : "+v"(x) : "v"(b));
      MH(u0) MH(u1) MH(u2) MH(u3) MH(u4) MH(u5) MH(u6) MH(u7)
    } else if (OP == 3) {  // v_mul_u32_u24
#define M24(x) asm volatile("v_mul_u32_u24 %0, %0, %1" : "+v"(x) : "v"(b));
      M24(u0) M24(u1) M24(u2) M24(u3) M24(u4) M24(u5) M24(u6) M24(u7)
    } else if (OP == 4) {  // v_fma_f64
#define F(x) asm volatile("v_fma_f64 %0, %0, %1, %2" : "+v"(x) : "v"(e), "v"(f));
      F(d0) F(d1) F(d2) F(d3) F(d4) F(d5) F(d6) F(d7)
    } else if (OP == 5) {  // v_add_u32
#define A(x) asm volatile("v_add_u32 %0, %0, %1" : "+v"(x) : "v"(b));
      A(u0) A(u1) A(u2) A(u3) A(u4) A(u5) A(u6) A(u7)
    } else if (OP == 6) {  // v_lshl_add_u64
#define LA(x) asm volatile("v_lshl_add_u64 %0, %0, 0, %1" : "+v"(x) : "v"(a0));
      LA(a1) LA(a2) LA(a3) LA(a4) LA(a5) LA(a6) LA(a7) LA(a1)
    } else if (OP == 7) {  // v_mul_hi_u32_u24
#define MH24(x) asm volatile("v_mul_hi_u32_u24 %0, %0, %1" : "+v"(x) : "v"(b));
      MH24(u0) MH24(u1) MH24(u2) MH24(u3) MH24(u4) MH24(u5) MH24(u6) MH24(u7)
    } else if (OP == 8) {  // v_mad_u32_u24
#define MA24(x) asm volatile("v_mad_u32_u24 %0, %0, %1, %2" : "+v"(x) : "v"(b), "v"(c));
      MA24(u0) MA24(u1) MA24(u2) MA24(u3) MA24(u4) MA24(u5) MA24(u6) MA24(u7)
    } else if (OP == 9) {  // v_sub_co_u32 + v_subb_co_u32 (64-bit sub pair)
#define SB(x) asm volatile("v_sub_co_u32 %0, vcc, %0, %1" : "+v"(x) : "v"(b) : "vcc");
      SB(u0) SB(u1) SB(u2) SB(u3) SB(u4) SB(u5) SB(u6) SB(u7)
    }
  }
  out[blockIdx.x * 256 + threadIdx.x] = a0 + a1 + a2 + a3 + a4+a5+a6+a7 + (uint64_t)(d0 + d1 + d2 + d3+d4+d5+d6+d7) + u0 + u1 + u2 + u3+u4+u5+u6+u7;
}
int main() {
  const int blocks = 256 * 32;
  uint64_t* out = nullptr;
  if (hipMalloc(&out, (size_t)blocks * 256 * 8) != hipSuccess) return 1;
  const char* names[] = {"v_mad_u64_u32", "v_mul_lo_u32", "v_mul_hi_u32", "v_mul_u32_u24", "v_fma_f64", "v_add_u32", "v_lshl_add_u64", "v_mul_hi_u32_u24", "v_mad_u32_u24", "v_sub_co_u32"};
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return 1;
  int clk = 0;
  (void)hipDeviceGetAttribute(&clk, hipDeviceAttributeClockRate, 0);
  int cus = 0;
  (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0);
  printf("clock %d kHz, CUs %d\n", clk, cus);
  for (int op = 0; op < 10; op++) {
    for (int rep = 0; rep < 2; rep++) {
      (void)hipEventRecord(e0);
      switch (op) {
        case 0: kern<0><<<blocks, 256>>>(out, 3); break; case 1: kern<1><<<blocks, 256>>>(out, 3); break;
        case 2: kern<2><<<blocks, 256>>>(out, 3); break; case 3: kern<3><<<blocks, 256>>>(out, 3); break;
        case 4: kern<4><<<blocks, 256>>>(out, 3); break; case 5: kern<5><<<blocks, 256>>>(out, 3); break;
        case 6: kern<6><<<blocks, 256>>>(out, 3); break; case 7: kern<7><<<blocks, 256>>>(out, 3); break;
        case 8: kern<8><<<blocks, 256>>>(out, 3); break; case 9: kern<9><<<blocks, 256>>>(out, 3); break;
      }
      (void)hipEventRecord(e1); (void)hipEventSynchronize(e1);
      float ms = 0; (void)hipEventElapsedTime(&ms, e0, e1);
      double lane_ops = (double)blocks * 256 * ITERS * 8;
      double per_s = lane_ops / (ms * 1e-3);
      // cycles per wave-instruction per SIMD: (cus*4 SIMDs * clk) / (wave instrs per s)
      double wave_instr_per_s = per_s / 64;
      double cyc = (double)cus * 4 * clk * 1e3 / wave_instr_per_s;
      if (rep) printf("%-18s %8.3f ms  %.3e lane-ops/s  %.2f cycles/wave-instr/SIMD\n", names[op], ms, per_s, cyc);
    }
  }
  return 0;
}
