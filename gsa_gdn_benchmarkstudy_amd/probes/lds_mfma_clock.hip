// Microbenchmark: MFMA rate and core clock on gfx950 with constant and with
// random operand data, alone and fed by ds_read_b128 operand reads.
//
// Not part of libgsa_hip.so.  The dense attention kernel issues about one
// ds_read_b128 per v_mfma_f32_32x32x16_bf16 (its K and V^T operands come from
// LDS) on random bf16 data; this probe separates what those reads cost in
// LDS bandwidth from what they cost in clock.
//
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       gsa_gdn_benchmarkstudy_amd/probes/lds_mfma_clock.hip -o /tmp/lds_mfma_clock
//   /tmp/lds_mfma_clock
//
// Grid: 256 blocks of 512 threads (two waves per SIMD), 64 KiB of LDS each.
// Every instruction of interest is inline asm.  Modes: MFMA only (two
// accumulator chains per wave, operands in registers); one read per MFMA
// (its A operand from LDS, four reads in flight); two reads per MFMA (A and B
// from LDS); reads only (eight in flight, no MFMA).  "const" data is 1.0 and
// 2^-7 everywhere, "rand" data random bf16 of magnitude 2^-7..2^-6 (with
// random signs in LDS).  Each line prints the best of three launches in ns per MFMA per SIMD
// and, from wave 0 of every block, the core clock over the loop: s_memtime
// cycles over s_memrealtime (100 MHz) ticks, averaged over the blocks of the
// last launch.
#include <hip/hip_runtime.h>
#include <cstdio>
typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
constexpr int kIters = 2048;

__device__ __forceinline__ unsigned hsh(unsigned x) { x ^= x >> 16; x *= 0x7feb352du; x ^= x >> 15; x *= 0x846ca68bu; x ^= x >> 16; return x; }

// MODE 0: MFMA only (A, B in registers), 4 per iteration, 2 chains
// MODE 1: 1 ds_read_b128 per MFMA (A from LDS)
// MODE 2: 2 ds_read_b128 per MFMA (A and B from LDS)
// MODE 3: reads only, 8 per iteration (no MFMA)
// RND: LDS and register data random (else constant 1.0 / 2^-7)
template <int MODE, bool RND>
__global__ __launch_bounds__(512, 1) void probe(float* out, unsigned long long* clk) {
  __shared__ u32x4 lds[4096];   // 64 KiB
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  for (int i = tid; i < 4096; i += 512) {
    u32x4 v;
    for (int j = 0; j < 4; ++j) {
      const unsigned h = hsh(i * 4 + j + 12345u);
      const unsigned lo = RND ? (0x3c00u | (h & 0x7fu) | ((h >> 8) & 0x8000u)) : 0x3f80u;
      const unsigned hi = RND ? (0x3c00u | ((h >> 16) & 0x7fu) | ((h >> 1) & 0x8000u)) : 0x3f80u;
      v[j] = lo | (hi << 16);
    }
    lds[i] = v;
  }
  __syncthreads();
  // conflict-free: 17-unit rows like the dense kernel's K tile
  const unsigned addr = (unsigned)(((lane & 31) * 17 + (lane >> 5) + w * 2) * 16);
  const unsigned base = (unsigned)(size_t)(const __attribute__((address_space(3))) void*)lds;
  const unsigned a0 = base + addr;
  floatx16 acc0, acc1;
  for (int r = 0; r < 16; ++r) { acc0[r] = 0.f; acc1[r] = 0.f; }
  u32x4 b, c;
  for (int j = 0; j < 4; ++j) {
    b[j] = RND ? (0x3c003c00u | (hsh(lane * 8 + j) & 0x007f007fu)) : 0x3c003c00u;
    c[j] = RND ? (0x3c003c00u | (hsh(lane * 8 + j + 4) & 0x007f007fu)) : 0x3f803f80u;
  }
  u32x4 o0, o1, o2, o3, o4, o5, o6, o7;
  o0 = o1 = o2 = o3 = o4 = o5 = o6 = o7 = c;
  const unsigned long long c0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < kIters; ++it) {
    if constexpr (MODE == 0) {
      asm volatile(
        "v_mfma_f32_32x32x16_bf16 %0, %2, %3, %0\n\tv_mfma_f32_32x32x16_bf16 %1, %3, %2, %1\n\t"
        "v_mfma_f32_32x32x16_bf16 %0, %2, %3, %0\n\tv_mfma_f32_32x32x16_bf16 %1, %3, %2, %1\n\t"
        : "+v"(acc0), "+v"(acc1) : "v"(c), "v"(b) : "memory");
    } else if constexpr (MODE == 1) {
      asm volatile(
        "ds_read_b128 %2, %7\n\tds_read_b128 %3, %7 offset:32\n\tds_read_b128 %4, %7 offset:64\n\t"
        "ds_read_b128 %5, %7 offset:96\n\ts_waitcnt lgkmcnt(3)\n\tv_mfma_f32_32x32x16_bf16 %0, %2, %6, %0\n\t"
        "s_waitcnt lgkmcnt(2)\n\tv_mfma_f32_32x32x16_bf16 %1, %3, %6, %1\n\t"
        "s_waitcnt lgkmcnt(1)\n\tv_mfma_f32_32x32x16_bf16 %0, %4, %6, %0\n\t"
        "s_waitcnt lgkmcnt(0)\n\tv_mfma_f32_32x32x16_bf16 %1, %5, %6, %1\n\t"
        : "+v"(acc0), "+v"(acc1), "=&v"(o0), "=&v"(o1), "=&v"(o2), "=&v"(o3) : "v"(b), "v"(a0) : "memory");
    } else if constexpr (MODE == 2) {
      asm volatile(
        "ds_read_b128 %2, %10\n\tds_read_b128 %3, %10 offset:2048\n\tds_read_b128 %4, %10 offset:32\n\t"
        "ds_read_b128 %5, %10 offset:2080\n\tds_read_b128 %6, %10 offset:64\n\tds_read_b128 %7, %10 offset:2112\n\t"
        "ds_read_b128 %8, %10 offset:96\n\tds_read_b128 %9, %10 offset:2144\n\t"
        "s_waitcnt lgkmcnt(6)\n\tv_mfma_f32_32x32x16_bf16 %0, %2, %3, %0\n\t"
        "s_waitcnt lgkmcnt(4)\n\tv_mfma_f32_32x32x16_bf16 %1, %4, %5, %1\n\t"
        "s_waitcnt lgkmcnt(2)\n\tv_mfma_f32_32x32x16_bf16 %0, %6, %7, %0\n\t"
        "s_waitcnt lgkmcnt(0)\n\tv_mfma_f32_32x32x16_bf16 %1, %8, %9, %1\n\t"
        : "+v"(acc0), "+v"(acc1), "=&v"(o0), "=&v"(o1), "=&v"(o2), "=&v"(o3), "=&v"(o4), "=&v"(o5), "=&v"(o6),
          "=&v"(o7) : "v"(a0) : "memory");
    } else {
      asm volatile(
        "ds_read_b128 %0, %8\n\tds_read_b128 %1, %8 offset:2048\n\tds_read_b128 %2, %8 offset:32\n\t"
        "ds_read_b128 %3, %8 offset:2080\n\tds_read_b128 %4, %8 offset:64\n\tds_read_b128 %5, %8 offset:2112\n\t"
        "ds_read_b128 %6, %8 offset:96\n\tds_read_b128 %7, %8 offset:2144\n\ts_waitcnt lgkmcnt(0)\n\t"
        : "=&v"(o0), "=&v"(o1), "=&v"(o2), "=&v"(o3), "=&v"(o4), "=&v"(o5), "=&v"(o6), "=&v"(o7) : "v"(a0) : "memory");
    }
  }
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
  const unsigned long long c1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  if (tid == 0) { clk[2 * blockIdx.x] = c1 - c0; clk[2 * blockIdx.x + 1] = r1 - r0; }
  float s = 0.f;
  for (int r = 0; r < 16; ++r) s += acc0[r] + acc1[r];
  out[blockIdx.x * 512 + tid] = s + (float)(o0[0] ^ o1[1] ^ o2[2] ^ o3[3] ^ o4[0] ^ o5[1] ^ o6[2] ^ o7[3]);
}

static unsigned long long* g_clk;
static double g_ghz;
template <int M, bool R>
float run(float* d) {
  hipEvent_t e0, e1;
  (void)hipEventCreate(&e0); (void)hipEventCreate(&e1);
  float best = 1e30f;
  for (int rep = 0; rep < 3; ++rep) {
    (void)hipEventRecord(e0);
    hipLaunchKernelGGL((probe<M, R>), dim3(256), dim3(512), 0, 0, d, g_clk);
    (void)hipEventRecord(e1); (void)hipEventSynchronize(e1);
    float ms; (void)hipEventElapsedTime(&ms, e0, e1);
    if (ms < best) best = ms;
  }
  (void)hipEventDestroy(e0); (void)hipEventDestroy(e1);
  unsigned long long h[512];
  (void)hipMemcpy(h, g_clk, sizeof(h), hipMemcpyDeviceToHost);
  double c = 0, r = 0;
  for (int i = 0; i < 256; ++i) { c += (double)h[2 * i]; r += (double)h[2 * i + 1]; }
  g_ghz = c / (r * 10.0);   // realtime at 100 MHz: r ticks = r*10 ns
  return best;
}
int main() {
  float* d;
  if (hipMalloc(&d, 256 * 512 * 4) != hipSuccess || hipMalloc(&g_clk, 512 * 8) != hipSuccess) return 1;
  for (int i = 0; i < 20; ++i) run<0, true>(d);
  const double per_simd = 2.0 * kIters * 4;   // MFMAs per SIMD (2 waves x 4 per iteration)
  const double rd_bytes_cu = 8.0 * kIters * 8 * 1024;   // mode 3: bytes read per CU
  for (int rep = 0; rep < 2; ++rep) {
    double g[7];
    float m0c = run<0, false>(d); g[0] = g_ghz;
    float m0r = run<0, true>(d); g[1] = g_ghz;
    float m1c = run<1, false>(d); g[2] = g_ghz;
    float m1r = run<1, true>(d); g[3] = g_ghz;
    float m2c = run<2, false>(d); g[4] = g_ghz;
    float m2r = run<2, true>(d); g[5] = g_ghz;
    float r3 = run<3, true>(d); g[6] = g_ghz;
    printf("core clock over the loop, GHz (last launch): %.3f %.3f | %.3f %.3f | %.3f %.3f | reads %.3f\n",
           g[0], g[1], g[2], g[3], g[4], g[5], g[6]);
    printf("ns per MFMA per SIMD -- MFMA only: const %.2f rand %.2f | 1 read/MFMA: const %.2f rand %.2f | "
           "2 reads/MFMA: const %.2f rand %.2f\n",
           m0c * 1e6 / per_simd, m0r * 1e6 / per_simd, m1c * 1e6 / per_simd, m1r * 1e6 / per_simd,
           m2c * 1e6 / per_simd, m2r * 1e6 / per_simd);
    printf("reads only: %.4f ms, %.1f bytes/ns per CU\n", r3, rd_bytes_cu / (r3 * 1e6));
  }
  return 0;
}
