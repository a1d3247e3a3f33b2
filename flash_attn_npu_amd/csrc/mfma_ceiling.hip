// mfma_ceiling: the dense bf16 MFMA rate that this GPU sustains, as a
// reference point for the attention kernel's roofline.
//
// Every SIMD runs two waves of back-to-back bf16 MFMAs, either
// v_mfma_f32_32x32x16_bf16 (four independent accumulator chains per wave, the
// attention kernel's instruction) or v_mfma_f32_16x16x32_bf16 (eight chains,
// two instructions per 32x32x16 in FLOPs), operands rotating over 8 register
// pairs loaded once from a buffer of random bf16 values (or zeros).  No memory
// traffic and no other instruction inside the loop, so the rate is bounded
// only by the matrix cores and by the clock the board allows under that load.
// Two more 32x32x16 forms answer questions about the tile body:
//   32x32x16-1chain   one wave per SIMD and a single accumulator chain (every
//                     MFMA reads the previous one's result as its C input),
//                     the shape of a 32-key S^T block summed over D;
//   32x32x16-shareb   the B operand shared by consecutive pairs of MFMAs (as
//                     the two key blocks of a tile share Q), against the
//                     default's new A and B on every instruction.
// Each wave also stamps s_memtime (shader clock) and s_memrealtime (100 MHz)
// around its loop, from which the mean shader clock of the run follows.  The
// grid fills every SIMD with its waves; the program refuses to run if the
// kernel's registers would not let them be resident at once.
//
//     flash_attn_npu_amd/mfma_ceiling [random|zero] [iterations]
//                                     [32x32x16|16x16x32|32x32x16-1chain|32x32x16-shareb]
//
// Built by flash_attn_npu_amd/build.py next to the library.
#include <hip/hip_runtime.h>

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;    // workgroups of 4 waves, one per SIMD
constexpr int kPairs = 8;        // operand register pairs per wave
constexpr size_t kSrcElems = 1u << 20;  // bf16x8 values in the operand buffer (16 MiB)
constexpr double kFlopPerIter = 16.0 * 2 * 32 * 32 * 16;  // 16 32x32x16 (or 32 16x16x32) per iteration

// SHAPE 32: 32x32x16 over CHAINS accumulators (SHAREB: B index advances every
// second MFMA); SHAPE 16: 16x16x32 over eight.  WPS waves per SIMD.
template <int SHAPE, int CHAINS, bool SHAREB, int WPS>
__global__ void __launch_bounds__(kThreads, WPS) mfma_loop(const bf16x8_t *src, float *sink, uint64_t *stamps,
                                                           int iters) {
  const int tid = blockIdx.x * blockDim.x + threadIdx.x;
  bf16x8_t a[kPairs], b[kPairs];
#pragma unroll
  for (int i = 0; i < kPairs; ++i) {
    a[i] = src[(size_t)(tid * 2 * kPairs + i) % kSrcElems];
    b[i] = src[(size_t)(tid * 2 * kPairs + kPairs + i) % kSrcElems];
  }
  float s = 0.f;
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
  if constexpr (SHAPE == 32) {
    f32x16_t c[CHAINS];
#pragma unroll
    for (int j = 0; j < CHAINS; ++j) c[j] = (f32x16_t){};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int bi = SHAREB ? ((i / 2) * 3 + 1) % kPairs : (3 * (i - i % 4) + i % 4) % kPairs;
        c[i % CHAINS] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i % kPairs], b[bi], c[i % CHAINS], 0, 0, 0);
      }
    }
#pragma unroll
    for (int j = 0; j < CHAINS; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) s += c[j][r];
  } else {
    f32x4_t c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = (f32x4_t){0.f, 0.f, 0.f, 0.f};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int i = 0; i < 32; ++i)
        c[i & 7] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i % kPairs], b[(i * 3 + i / kPairs) % kPairs], c[i & 7], 0,
                                                           0, 0);
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) s += c[j][0] + c[j][1] + c[j][2] + c[j][3];
  }
  const uint64_t t1 = __builtin_amdgcn_s_memtime();
  const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
  sink[tid] = s;  // keeps the loop live
  if ((threadIdx.x & 63) == 0) {
    const int w = tid / 64;
    stamps[2 * w] = t1 - t0;
    stamps[2 * w + 1] = r1 - r0;
  }
}

static int check(hipError_t e, const char *what) {
  if (e != hipSuccess) {
    fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
    return 1;
  }
  return 0;
}

int main(int argc, char **argv) {
  const bool zero = argc > 1 && strcmp(argv[1], "zero") == 0;
  const int iters = argc > 2 ? atoi(argv[2]) : 1000000;
  const char *shape_name = argc > 3 ? argv[3] : "32x32x16";
  if (iters < 1) {
    fprintf(stderr, "iterations must be >= 1\n");
    return 2;
  }
  void (*kern)(const bf16x8_t *, float *, uint64_t *, int) = nullptr;
  int wps = 2;  // waves per SIMD = workgroups per CU
  bool small = false;
  if (strcmp(shape_name, "32x32x16") == 0) {
    kern = mfma_loop<32, 4, false, 2>;
  } else if (strcmp(shape_name, "16x16x32") == 0) {
    kern = mfma_loop<16, 8, false, 2>;
    small = true;
  } else if (strcmp(shape_name, "32x32x16-1chain") == 0) {
    kern = mfma_loop<32, 1, false, 1>;
    wps = 1;
  } else if (strcmp(shape_name, "32x32x16-shareb") == 0) {
    kern = mfma_loop<32, 4, true, 2>;
  } else {
    fprintf(stderr, "shape must be 32x32x16, 16x16x32, 32x32x16-1chain or 32x32x16-shareb\n");
    return 2;
  }
  int dev = 0, cus = 0, resident = 0;
  if (check(hipGetDevice(&dev), "hipGetDevice") ||
      check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "CU count") ||
      check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&resident, kern, kThreads, 0), "occupancy"))
    return 1;
  if (resident < wps) {
    fprintf(stderr, "only %d workgroups of this kernel fit on a CU, %d needed\n", resident, wps);
    return 1;
  }
  const int blocks = cus * wps;
  const int waves = blocks * kThreads / 64;
  bf16x8_t *src = nullptr;
  float *sink = nullptr;
  uint64_t *stamps = nullptr;
  if (check(hipMalloc(&src, kSrcElems * sizeof(bf16x8_t)), "hipMalloc") ||
      check(hipMalloc(&sink, (size_t)blocks * kThreads * sizeof(float)), "hipMalloc") ||
      check(hipMalloc(&stamps, (size_t)waves * 2 * sizeof(uint64_t)), "hipMalloc"))
    return 1;
  bf16x8_t *host = (bf16x8_t *)malloc(kSrcElems * sizeof(bf16x8_t));
  uint64_t *hst = (uint64_t *)malloc((size_t)waves * 2 * sizeof(uint64_t));
  if (host == nullptr || hst == nullptr) return 1;
  uint32_t lcg = 12345u;  // uniform values in [-1, 1)
  for (size_t i = 0; i < kSrcElems; ++i)
    for (int j = 0; j < 8; ++j) {
      lcg = lcg * 1664525u + 1013904223u;
      host[i][j] = (__bf16)(zero ? 0.f : ((float)(lcg >> 8) / 16777216.f - 0.5f) * 2.f);
    }
  if (check(hipMemcpy(src, host, kSrcElems * sizeof(bf16x8_t), hipMemcpyHostToDevice), "hipMemcpy")) return 1;
  hipEvent_t e0, e1;
  if (check(hipEventCreate(&e0), "event") || check(hipEventCreate(&e1), "event")) return 1;
  hipLaunchKernelGGL(kern, dim3(blocks), dim3(kThreads), 0, 0, src, sink, stamps, 100);
  if (check(hipDeviceSynchronize(), "warmup")) return 1;
  printf("%d CUs, %d waves (%d per SIMD), v_mfma_f32_%s_bf16, %s operands, %d iterations of %d MFMAs per wave\n",
         cus, waves, wps, shape_name, zero ? "zero" : "random", iters, small ? 32 : 16);
  for (int rep = 0; rep < 4; ++rep) {
    if (check(hipEventRecord(e0, 0), "event record")) return 1;
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(kThreads), 0, 0, src, sink, stamps, iters);
    if (check(hipEventRecord(e1, 0), "event record") || check(hipEventSynchronize(e1), "run")) return 1;
    float ms = 0.f;
    if (check(hipEventElapsedTime(&ms, e0, e1), "elapsed")) return 1;
    if (check(hipMemcpy(hst, stamps, (size_t)waves * 2 * sizeof(uint64_t), hipMemcpyDeviceToHost), "stamps"))
      return 1;
    double clk = 0.0;
    for (int w = 0; w < waves; ++w) clk += (double)hst[2 * w] / ((double)hst[2 * w + 1] / 100e6);
    clk /= waves;
    const double flops = (double)waves * iters * kFlopPerIter;
    printf("run %d: %.1f ms, %.1f TFLOP/s, mean shader clock %.0f MHz\n", rep, ms, flops / (ms * 1e-3) / 1e12,
           clk / 1e6);
    fflush(stdout);
  }
  return 0;
}
