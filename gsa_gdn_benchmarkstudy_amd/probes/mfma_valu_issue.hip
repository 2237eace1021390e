// Microbenchmark: how MFMA and VALU instructions share a gfx950 SIMD.
//
// Not part of libgsa_hip.so.  The dense attention kernel's design notes rest
// on these figures: a v_mfma_f32_32x32x16_bf16 holds the matrix core for 32
// cycles, and the question is how much VALU work (the softmax's fma, exp,
// max, pack and row-sum instructions) can run beside it for free -- from the
// same wave, from another wave of the same SIMD, and with the accumulators in
// arch VGPRs or in AGPRs.
//
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       gsa_gdn_benchmarkstudy_amd/probes/mfma_valu_issue.hip -o /tmp/mfma_valu_issue
//   /tmp/mfma_valu_issue
//
// Grid: 256 blocks of 512 threads, one block per CU, two waves per SIMD.  Every
// instruction of interest is inline asm, so the listing is exactly the loop
// below; the VALU work is 8 independent fma (or exp) chains per lane, never
// dependent on an MFMA result.  Each line prints the best of three launches
// and the time per "MFMA slot" = one MFMA instruction per SIMD in the
// MFMA-only configuration.  Modes:
//   mfma     every wave: 4 independent accumulator chains of MFMAs
//   fused n  every wave: each MFMA followed by n VALU instructions
//   valu n   every wave: only the n VALU instructions per slot
//   alone/split  waves 0-3 (one per SIMD) run MFMAs, waves 4-7 VALU; "alone"
//            runs one side with the other side idle
#include <hip/hip_runtime.h>

#include <cstdio>

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
constexpr int kIters = 2048;

template <bool AG>
__device__ __forceinline__ void mfma(floatx16& acc, const bf16x8& a, const bf16x8& b) {
  if constexpr (AG) asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
  else asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void valu(float& x, float c1, float c2, bool exp) {
  if (exp) asm volatile("v_exp_f32 %0, %0" : "+v"(x));
  else asm volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(x) : "v"(c1), "v"(c2));
}

// MODE 0: MFMA only; 1: MFMA + K VALU per MFMA (same wave); 2: VALU only (K per slot);
// 3: waves 0-3 MFMA, waves 4-7 2K VALU per slot; 4: waves 0-3 MFMA, 4-7 idle;
// 5: waves 0-3 idle, 4-7 2K VALU per slot.  E: every K-th VALU is an exp.
template <int MODE, bool AG, int K, bool E>
__global__ __launch_bounds__(512, 1) void probe(float* out, float c1, float c2) {
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  bf16x8 a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)(0.001f * (lane + i));
    b[i] = (__bf16)(0.002f * (lane - i));
  }
  floatx16 acc[4];
  for (int j = 0; j < 4; ++j)
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.f;
  float x[8];
  for (int i = 0; i < 8; ++i) x[i] = 0.1f * (lane + i);
  const bool do_m = MODE == 0 || MODE == 1 || ((MODE == 3 || MODE == 4) && w < 4);
  const bool do_v = MODE == 1 || MODE == 2 || ((MODE == 3 || MODE == 5) && w >= 4);
  const int nv = (MODE == 3 || MODE == 5) ? 2 * K : K;
  if (do_m && !do_v) {
    for (int it = 0; it < kIters; ++it)
#pragma unroll
      for (int j = 0; j < 4; ++j) mfma<AG>(acc[j], a, b);
  } else if (do_m && do_v) {
    for (int it = 0; it < kIters; ++it)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        mfma<AG>(acc[j], a, b);
#pragma unroll
        for (int k = 0; k < K; ++k) valu(x[(j * K + k) & 7], c1, c2, E && k == K - 1);
      }
  } else if (do_v) {
    for (int it = 0; it < kIters; ++it)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        for (int k = 0; k < nv; ++k) valu(x[(j * K + k) & 7], c1, c2, E && (k % K) == K - 1);
  }
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  float s = 0.f;
  for (int i = 0; i < 8; ++i) s += x[i];
  for (int j = 0; j < 4; ++j)
    for (int r = 0; r < 16; ++r) s += acc[j][r];
  out[blockIdx.x * 512 + tid] = s;
}

static float* g_out;

template <int MODE, bool AG, int K, bool E>
float run() {
  hipEvent_t e0, e1;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return -1.f;
  float best = 1e30f;
  for (int rep = 0; rep < 3; ++rep) {
    if (hipEventRecord(e0) != hipSuccess) return -1.f;
    hipLaunchKernelGGL((probe<MODE, AG, K, E>), dim3(256), dim3(512), 0, 0, g_out, 0.999f, 0.001f);
    if (hipEventRecord(e1) != hipSuccess || hipEventSynchronize(e1) != hipSuccess) return -1.f;
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, e0, e1) != hipSuccess) return -1.f;
    if (ms < best) best = ms;
  }
  (void)hipEventDestroy(e0);
  (void)hipEventDestroy(e1);
  return best;
}

int main() {
  if (hipMalloc(&g_out, 256 * 512 * sizeof(float)) != hipSuccess) return 1;
  for (int i = 0; i < 20; ++i) run<0, false, 4, false>();   // clocks settle
  const double slots = 256.0 * 8 * kIters * 4 / 1024;        // MFMA instructions per SIMD, mode 0
  auto pr = [&](const char* name, float ms) {
    printf("%-44s %.4f ms  %6.2f ns per MFMA slot per SIMD\n", name, ms, ms * 1e6 / slots);
  };
  pr("mfma (VGPR accumulators)", run<0, false, 4, false>());
  pr("mfma (AGPR accumulators)", run<0, true, 4, false>());
  pr("valu 4 fma", run<2, false, 4, false>());
  pr("valu 3 fma + 1 exp", run<2, false, 4, true>());
  pr("fused 1 fma", run<1, false, 1, false>());
  pr("fused 2 fma", run<1, false, 2, false>());
  pr("fused 4 fma", run<1, false, 4, false>());
  pr("fused 4 fma, AGPR accumulators", run<1, true, 4, false>());
  pr("fused 3 fma + 1 exp", run<1, false, 4, true>());
  pr("fused 8 fma", run<1, false, 8, false>());
  pr("alone: MFMA waves (1/SIMD)", run<4, false, 4, false>());
  pr("alone: VALU waves (1/SIMD), 8 fma", run<5, false, 4, false>());
  pr("split: both, 8 fma", run<3, false, 4, false>());
  pr("alone: VALU waves (1/SIMD), 4 fma", run<5, false, 2, false>());
  pr("split: both, 4 fma", run<3, false, 2, false>());
  pr("alone: VALU waves (1/SIMD), 2 fma", run<5, false, 1, false>());
  pr("split: both, 2 fma", run<3, false, 1, false>());
  pr("alone: VALU waves (1/SIMD), 6 fma + 2 exp", run<5, false, 4, true>());
  pr("split: both, 6 fma + 2 exp", run<3, false, 4, true>());
  (void)hipFree(g_out);
  return 0;
}
