// probe_mfma_rate.hip -- standalone measurement of the v_mfma_f32_32x32x16_bf16 issue rate on one
// MI355X, against the waves each SIMD holds.  Not part of libsta_hip.so: it puts the score
// kernel's MFMA figures in context (the rate the matrix pipes sustain on random bf16 operands,
// where the chip lowers its clock under load, and how it depends on occupancy).
//
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//         -mllvm -amdgpu-mfma-vgpr-form=1 -o probe_mfma_rate probe_mfma_rate.hip
//
// With -DAGPR_A the A operands are held in AGPRs (as the score kernel holds its Q fragments):
// each k step's operands are pinned there by an empty asm, which adds no instruction to the loop.
//
// Every wave runs chains of 24 dependent products (the score kernel's pass 2 issues three
// products per k step, eight k steps per 32-key block, into one accumulator) on operands drawn
// from a per-lane xorshift generator, so the data toggles as real scores do.  96 KB of LDS per
// workgroup pins one workgroup to a CU: WAVES / 4 waves per SIMD.  768 workgroups, as pass 2 at
// config 1 launches.  Printed: ms and the issued rate as a fraction of the 2.5 PFLOP/s peak.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef float floatx16 __attribute__((ext_vector_type(16)));

template <int CHAINS, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void mfma_rate_kernel(float* out, int iters, uint32_t seed) {
  __shared__ float pad[24 * 1024];
  pad[threadIdx.x] = (float)seed;
  __syncthreads();
  uint32_t hs = (blockIdx.x * 1024u + threadIdx.x) * 2654435761u + (uint32_t)pad[(threadIdx.x + 1) % (64 * WAVES)];
  auto rnd = [&]() {
    hs ^= hs << 13;
    hs ^= hs >> 17;
    hs ^= hs << 5;
    return ((float)(hs & 0xffff) / 32768.0f - 1.0f) * 2.0f;
  };
  bf16x8 a[8], b[2];
  for (int i = 0; i < 8; ++i)
    for (int j = 0; j < 8; ++j) a[i][j] = (__bf16)rnd();
  for (int j = 0; j < 8; ++j) {
    b[0][j] = (__bf16)rnd();
    b[1][j] = (__bf16)rnd();
  }
  floatx16 acc[CHAINS];
  for (int c = 0; c < CHAINS; ++c) acc[c] = floatx16{};
  for (int it = 0; it < iters; ++it) {
#ifdef AGPR_A
#pragma unroll
    for (int i = 0; i < 8; ++i) asm volatile("" : "+a"(a[i]));
#endif
#pragma unroll
    for (int s = 0; s < 24 / CHAINS; ++s)
#pragma unroll
      for (int c = 0; c < CHAINS; ++c)
        acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[(s + c) & 7], b[s & 1], acc[c], 0, 0, 0);
  }
  float r = 0.0f;
  for (int c = 0; c < CHAINS; ++c)
    for (int i = 0; i < 16; ++i) r += acc[c][i];
  out[blockIdx.x * blockDim.x + threadIdx.x] = r;
}

#define CHECK(x)                                                                   \
  do {                                                                             \
    hipError_t e_ = (x);                                                           \
    if (e_ != hipSuccess) {                                                        \
      fprintf(stderr, "%s failed: %s\n", #x, hipGetErrorString(e_));               \
      exit(1);                                                                     \
    }                                                                              \
  } while (0)

template <int CHAINS, int WAVES>
void run(int iters_per_wave_total) {
  const int nwg = 768;
  const int iters = iters_per_wave_total / WAVES;   // the same total work for every shape
  float* out;
  CHECK(hipMalloc(&out, (size_t)nwg * 64 * WAVES * sizeof(float)));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  float best = 1e30f;
  for (int rep = 0; rep < 4; ++rep) {   // the first launches also ramp the clock
    CHECK(hipEventRecord(e0));
    mfma_rate_kernel<CHAINS, WAVES><<<nwg, 64 * WAVES>>>(out, iters, 12345u + rep);
    CHECK(hipEventRecord(e1));
    CHECK(hipEventSynchronize(e1));
    float ms;
    CHECK(hipEventElapsedTime(&ms, e0, e1));
    best = ms < best ? ms : best;
  }
  const double flops = (double)nwg * WAVES * iters * 24 * 32 * 32 * 16 * 2;
  printf("waves/SIMD %d  chains/wave %d: %.3f ms  %.0f TFLOP/s issued  %.1f%% of 2.5 PFLOP/s\n", WAVES / 4, CHAINS,
         best, flops / best / 1e9, flops / best / 1e9 / 2500.0 * 100.0);
  CHECK(hipFree(out));
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
}

int main() {
  const int total = 5600;   // iterations x waves per workgroup
  run<1, 4>(total);
  run<2, 4>(total);
  run<1, 8>(total);
  run<2, 8>(total);
  run<1, 12>(total);
  run<1, 16>(total);
  return 0;
}
