// Issue-rate microbenchmark of gfx950: how much VALU work a SIMD hides behind
// v_mfma_f32_32x32x16_bf16 products.
//
// Each wave runs `iters` iterations of: NM MFMAs in four independent accumulator chains, NE
// v_exp_f32, NF v_fma_f32 and NC v_cvt_pk_bf16_f32 on registers the MFMAs do not touch, with
// sched_group_barrier interleaving one MFMA with an even share of the VALU instructions (the
// pattern the flash kernels use).  The shader clock counter (s_memtime) brackets the loop in
// every wave; the reported figure is loop cycles / iters for the slowest wave, i.e. the cycles
// a SIMD spends per iteration of each of its W resident waves.  With no overlap between the
// two pipes a mixed variant would take the sum of its MFMA-only and VALU-only rows; with full
// overlap, the larger of the two.
//
// Build and run (one MI355X):
//   hipcc -O3 --offload-arch=gfx950 -Xclang -target-feature -Xclang -packed-fp32-ops \
//         -o /tmp/coexec pope-pytorch_amd/microbench/mfma_valu_coexec.cpp && /tmp/coexec
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>

#define CHECK(x)                                                              \
  do {                                                                        \
    hipError_t e_ = (x);                                                      \
    if (e_ != hipSuccess) {                                                   \
      fprintf(stderr, "%s:%d %s\n", __FILE__, __LINE__, hipGetErrorString(e_)); \
      exit(1);                                                                \
    }                                                                         \
  } while (0)

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(16))) float f32x16;

template <int NM, int NE, int NF, int NC>
__global__ __launch_bounds__(256) void coexec(float* out, unsigned long long* cyc, int iters) {
  f32x16 c[4] = {};
  bf16x8 a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)(threadIdx.x * 0.001f);
    b[i] = (__bf16)(i * 0.01f);
  }
  float e[16 + 1], f[32 + 1], g[32 + 1];
  unsigned int pk[16 + 1];
  for (int i = 0; i < 17; ++i) e[i] = threadIdx.x * 1e-3f - i;
  for (int i = 0; i < 33; ++i) f[i] = threadIdx.x * 1e-3f + i;
  for (int i = 0; i < 33; ++i) g[i] = threadIdx.x * 2e-3f - i;
  for (int i = 0; i < 17; ++i) pk[i] = 0;
  __syncthreads();
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < NM; ++j) c[j & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c[j & 3], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < NE; ++i) e[i] = __builtin_amdgcn_exp2f(e[i]);
#pragma unroll
    for (int i = 0; i < NF; ++i) f[i] = __builtin_fmaf(f[i], 0.999f, 0.25f);
#pragma unroll
    for (int i = 0; i < NC; ++i) {
      asm volatile("" : "+v"(g[2 * i]), "+v"(g[2 * i + 1]));   // new inputs every iteration
      bf16x2 v = {(__bf16)g[2 * i], (__bf16)g[2 * i + 1]};
      pk[i] ^= __builtin_bit_cast(unsigned int, v);
    }
    if constexpr (NM > 0 && NE + NF + NC > 0) {
      constexpr int V = NE + NF + 2 * NC;   // VALU instructions per iteration (cvt + xor)
      constexpr int PER = (V + NM - 1) / NM;
#pragma unroll
      for (int j = 0; j < NM; ++j) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, PER, 0);
      }
    }
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  float s = 0;
  for (int j = 0; j < 4; ++j)
    for (int i = 0; i < 16; ++i) s += c[j][i];
  for (int i = 0; i < 16; ++i) s += e[i] + (float)pk[i];
  for (int i = 0; i < 32; ++i) s += f[i];
  out[blockIdx.x * 256 + threadIdx.x] = s;
  if ((threadIdx.x & 63) == 0) atomicMax(cyc, t1 - t0);
}

template <int NM, int NE, int NF, int NC>
void run(float* out, unsigned long long* cyc, const char* name) {
  int dev = 0, cus = 0;
  CHECK(hipGetDevice(&dev));
  CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  const int iters = 4096;
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  printf("| %-34s |", name);
  double ghz = 0;
  for (int waves = 1; waves <= 2; ++waves) {
    // 256 threads = one wave per SIMD; W workgroups per CU give W waves per SIMD
    const int blocks = cus * waves;
    coexec<NM, NE, NF, NC><<<blocks, 256>>>(out, cyc, 16);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    CHECK(hipMemset(cyc, 0, 8));
    CHECK(hipEventRecord(e0));
    coexec<NM, NE, NF, NC><<<blocks, 256>>>(out, cyc, iters);
    CHECK(hipGetLastError());
    CHECK(hipEventRecord(e1));
    CHECK(hipEventSynchronize(e1));
    float ms = 0;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    unsigned long long c = 0;
    CHECK(hipMemcpy(&c, cyc, 8, hipMemcpyDeviceToHost));
    printf(" %8.1f |", (double)c / iters);
    ghz = (double)c / (ms * 1e6);
  }
  printf(" %5.2f |\n", ghz);
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
}

int main() {
  float* out;
  unsigned long long* cyc;
  CHECK(hipMalloc(&out, 4096 * 256 * 4));
  CHECK(hipMalloc(&cyc, 8));
  printf("shader-clock cycles per iteration of each wave (slowest wave), W waves per SIMD;\n"
         "clock = counter cycles / kernel time of the W = 2 run\n\n");
  printf("| %-34s | %8s | %8s | %5s |\n", "per iteration", "W = 1", "W = 2", "GHz");
  printf("|---|---|---|---|\n");
  run<8, 0, 0, 0>(out, cyc, "8 mfma");
  run<0, 16, 0, 0>(out, cyc, "16 exp");
  run<0, 0, 32, 0>(out, cyc, "32 fma");
  run<0, 0, 0, 16>(out, cyc, "16 cvt_pk_bf16 (+16 xor)");
  run<8, 16, 0, 0>(out, cyc, "8 mfma + 16 exp");
  run<8, 0, 32, 0>(out, cyc, "8 mfma + 32 fma");
  run<8, 0, 0, 16>(out, cyc, "8 mfma + 16 cvt_pk (+16 xor)");
  run<0, 16, 32, 8>(out, cyc, "16 exp + 32 fma + 8 cvt_pk");
  run<8, 16, 32, 8>(out, cyc, "8 mfma + 16 exp + 32 fma + 8 cvt");
  run<16, 16, 32, 8>(out, cyc, "16 mfma + 16 exp + 32 fma + 8 cvt");
  CHECK(hipFree(out));
  CHECK(hipFree(cyc));
  return 0;
}
