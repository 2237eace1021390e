// Main projection GEMM with the producer in its epilogue (gfx950 MFMA).
//
//   P = x W^T + b   for the q, k, v, value-gate and output-gate rows of the
//   fused projection weight, and straight from the accumulators:
//     q, og    -> bf16(P) rows (strided)
//     k        -> RoPE(bf16(P_k))                          [B,T,H,128]
//     v, vg    -> (bf16(P_v) * bf16(sigmoid(bf16(P_vg))))^T  [B,H,128,ldv]
//   so the projection output is never written whole and no producer pass
//   reads it back.  Same values as the projection GEMM followed by the
//   RoPE / value-gate producer: every step rounds to bf16 where that path
//   does.
//
// Weight layout ("packed", built once by gsa_proj_pack): the 5D weight rows
// are permuted so that one 256-column tile holds one kind of output and each
// wave's 64 columns hold both operands of its elementwise step:
//   q   tiles:  q rows in order
//   k   tiles:  per head, 32-row chunks in order d[0:32], d[64:96], d[32:64],
//               d[96:128] -> a wave holds d and its RoPE partner d+64
//   v/vg tiles: one head per tile, chunks v[0:32], vg[0:32], v[32:64], ...
//               -> a wave holds v[d] and vg[d]
//   og  tiles:  og rows in order
// and stored as 16 KiB tiles (256 rows x 32 k), each already in the LDS
// order the kernel reads (16-byte chunk c of row r at unit c ^ ((r>>2)&3)),
// so every weight load is one contiguous KiB per instruction.
//
// Kernel: persistent, one block of 8 waves per CU; tiles of 256 tokens x 256
// columns; waves 2 (tokens) x 4 (columns) of 128 x 64; K in steps of 32
// through a 4-stage LDS ring filled by direct global->LDS loads; one barrier
// per step, in its middle, after which the step's second half reads the next
// stage.  Tiles are dealt out per XCD (blocks b, b+8, ... share an XCD and
// its L2) in groups of 4 token tiles.  The q/k/og tiles use the transposed
// product (lane = token, 4 consecutive columns per register quad: 8-byte row
// stores); the v/vg tiles the direct one (lane = column, 4 consecutive tokens
// per quad: 8-byte stores along V^T's rows).
#include "gsa_common.h"

namespace gsa {
namespace proj {

constexpr int kBM = 256, kBN = 256, kBK = 32;
constexpr int kStages = 4;
constexpr int kNW = 8;                  // waves: 2 along tokens x 4 along columns
constexpr int kWN = 4;
constexpr int kIM = 4, kJN = 2;         // 32x32 MFMA tiles per wave: 128 tokens x 64 columns
constexpr int kDI = 16 / kNW;           // DMA instructions per wave, operand tile and stage
constexpr int kRowU = 4;                // 16-byte units per LDS row (32 bf16)
constexpr int kTileU = 256 * kRowU;     // one operand tile of a stage: 16 KiB
constexpr int kStageU = 2 * kTileU;     // token rows, then weight rows
constexpr size_t kLds = (size_t)kStages * kStageU * 16;   // 128 KiB
constexpr int kGroupM = 4;              // token tiles per group of the tile order

enum Kind { kQ = 0, kK = 1, kV = 2, kOG = 3 };

struct Args {
  const uint16_t* x; int64_t x_st;           // [M, D] token rows
  const uint16_t* w;                         // packed weight
  const float* bias;                         // packed bias [5D]
  const uint16_t* cos; const uint16_t* sin; int64_t cs_st;
  uint16_t* q; int64_t q_st;
  uint16_t* og; int64_t og_st;
  uint16_t* k_out;                           // [M, D]
  uint16_t* vt; int64_t vt_sb; int ldv;      // [B, H, 128, ldv]
  int M, T, D, nq;                           // nq = D / 256 tiles per D columns
};

// Source row (in q, k, v, vg, og order) of packed weight row n.
__host__ __device__ inline int packed_source_row(int n, int D) {
  if (n < D || n >= 4 * D) return n;                       // q, og
  if (n < 2 * D) {                                         // k
    const int l = n - D, head = l >> 7, c = (l >> 5) & 3;
    const int d = (c & 1) * 64 + (c >> 1) * 32 + (l & 31);
    return D + head * 128 + d;
  }
  const int l = n - 2 * D, head = l >> 8, c = (l >> 5) & 7;   // v / vg
  const int d = (c >> 1) * 32 + (l & 31);
  return ((c & 1) ? 3 * D : 2 * D) + head * 128 + d;
}

__global__ __launch_bounds__(256) void pack_kernel(const uint16_t* __restrict__ w, int64_t w_st,
                                                   const uint16_t* __restrict__ bias, int D,
                                                   uint16_t* __restrict__ wp, float* __restrict__ bp) {
  const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;   // packed 16-byte unit
  const int nks = D / kBK;
  const int64_t units = (int64_t)5 * D * D / 8;
  if (u < units) {
    const int64_t per_bn = (int64_t)nks * kTileU;
    const int bn = (int)(u / per_bn);
    const int rem = (int)(u - (int64_t)bn * per_bn);
    const int ks = rem / kTileU, wi = rem % kTileU;
    const int r = wi >> 2, p = wi & 3, c = p ^ ((r >> 2) & 3);
    const int src = packed_source_row(bn * kBN + r, D);
    const u32x4 v = *reinterpret_cast<const u32x4*>(w + (int64_t)src * w_st + ks * kBK + c * 8);
    *reinterpret_cast<u32x4*>(wp + u * 8) = v;
  }
  if (u < 5 * D) bp[u] = bias ? bf16lo(bias[packed_source_row((int)u, D)]) : 0.f;
}

#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
// Direct global -> LDS load: each lane's 16 bytes at base + voff land at
// lds + 16 * lane.  Completion is awaited with explicit vmcnt waits.  The
// s_nop is the wait state an LDS DMA needs after the SALU write of m0.
__device__ __forceinline__ void load_lds16(const void* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// s_waitcnt vmcnt(N) (gfx9 encoding, N < 64); expcnt and lgkmcnt not waited.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

__device__ __forceinline__ void tile_coords(int t, int ntm, int ntn, int& bm, int& bn) {
  const int g = t / (kGroupM * ntn), r = t - g * kGroupM * ntn;
  const int gm = min(kGroupM, ntm - kGroupM * g);
  bm = kGroupM * g + r % gm;
  bn = r / gm;
}

typedef float floatx16 __attribute__((ext_vector_type(16)));

struct Frag {
  floatx16 acc[kIM][kJN];
  bf16x8 a[2][kIM], b[2][kJN];
};

// MFMAs of one 16-deep step from operand buffer `buf`.  kT: transposed
// product (weight rows as the A operand): lane = token.
template <bool kT>
__device__ __forceinline__ void mm(Frag& f, int buf) {
#pragma unroll
  for (int i = 0; i < kIM; ++i)
#pragma unroll
    for (int j = 0; j < kJN; ++j)
      f.acc[i][j] = kT ? __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.b[buf][j], f.a[buf][i], f.acc[i][j], 0, 0, 0)
                       : __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[buf][i], f.b[buf][j], f.acc[i][j], 0, 0, 0);
}

// One LDS read interleaved between every MFMA pair... (6 reads, 8 MFMAs per step)
__device__ __forceinline__ void interleave() {
#pragma unroll
  for (int q = 0; q < kIM + kJN; ++q) {
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // DS read
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
  }
  __builtin_amdgcn_sched_group_barrier(0x008, kIM * kJN - (kIM + kJN), 0);
}

// Main loop over K for one tile.  On entry stages 0..kStages-2 are in flight
// (issued by the caller); on exit every LDS read of the tile is complete.
template <bool kT, typename Issue, typename Read>
__device__ __forceinline__ void tile_main(Frag& f, int nks, Issue&& issue, Read&& rd, int p0, int p1) {
#pragma unroll
  for (int i = 0; i < kIM; ++i)
#pragma unroll
    for (int j = 0; j < kJN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) f.acc[i][j][r] = 0.f;
  wait_vm<2 * kDI * (kStages - 2)>();          // stage 0 landed (this wave's loads)
  asm volatile("s_barrier" ::: "memory");       // ... and every wave's
  rd(0, p0, 0);
  for (int ks = 0; ks < nks - 1; ++ks) {
    rd(ks, p1, 1);                              // second 16 of stage ks
    mm<kT>(f, 0);
    interleave();
    __builtin_amdgcn_sched_barrier(0);
    // stage ks+1 complete for every wave; the slot of stage ks-1 is free
    if (ks + kStages - 2 < nks) wait_vm<2 * kDI * (kStages - 3)>(); else wait_vm<0>();
    asm volatile("s_barrier" ::: "memory");
    if (ks + kStages - 1 < nks) issue(ks + kStages - 1);
    __builtin_amdgcn_sched_barrier(0);
    rd(ks + 1, p0, 0);                          // first 16 of stage ks+1
    mm<kT>(f, 1);
    interleave();
    __builtin_amdgcn_sched_barrier(0);
  }
  rd(nks - 1, p1, 1);
  mm<kT>(f, 0);
  __builtin_amdgcn_sched_barrier(0);
  mm<kT>(f, 1);
}

__device__ __forceinline__ void store4(uint16_t* p, float a, float b, float c, float d) {
  uint2 v;
  v.x = pack_bf16(a, b);
  v.y = pack_bf16(c, d);
  *reinterpret_cast<uint2*>(p) = v;
}
__device__ __forceinline__ void load4(const uint16_t* p, float (&x)[4]) {
  const uint2 v = *reinterpret_cast<const uint2*>(p);
  x[0] = bf16lo(v.x); x[1] = bf16hi(v.x); x[2] = bf16lo(v.y); x[3] = bf16hi(v.y);
}

__global__ __launch_bounds__(64 * kNW, 1) void proj_fused_kernel(Args p) {
  extern __shared__ __align__(16) u32x4 dsm[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wu = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wu / kWN, wn = wu % kWN;
  const int i32 = lane & 31, h = lane >> 5;
  const int ntm = (p.M + kBM - 1) / kBM, ntn = 5 * p.nq, nt = ntm * ntn;
  const int nks = p.D / kBK;
  // blocks b, b+8, ... run on one XCD: XCD x owns tiles [x*per, (x+1)*per)
  const int per = (nt + 7) / 8, xcd = blockIdx.x & 7, gx = gridDim.x >> 3;
  const int tend = min(nt, xcd * per + per);
  int t = xcd * per + (int)(blockIdx.x >> 3);
  if (t >= tend) return;
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(dsm));

  // DMA: instruction n of wave wu fills LDS units (8n + wu)*64 .. +63 of an
  // operand tile: row u/4, stored unit u%4 holding chunk (u%4) ^ ((row>>2)&3).
  uint32_t xrow[kDI], xchunk[kDI];
#pragma unroll
  for (int n = 0; n < kDI; ++n) {
    const int u = (kNW * n + wu) * 64 + lane, row = u >> 2;
    xrow[n] = (uint32_t)row;
    xchunk[n] = (uint32_t)(((u & 3) ^ ((row >> 2) & 3)) * 16);
  }
  uint32_t xoff[kDI];
  const char* xa = nullptr;
  const char* wb = nullptr;
  auto issue = [&](int ks) {
    const uint32_t base = lds0 + (uint32_t)((ks % kStages) * kStageU * 16);
#pragma unroll
    for (int n = 0; n < kDI; ++n) {
      load_lds16(xa + ks * kBK * 2, xoff[n], base + (kNW * n + wu) * 1024);
      load_lds16(wb + (int64_t)ks * (kTileU * 16), (uint32_t)(((kNW * n + wu) * 64 + lane) * 16),
                 base + kTileU * 16 + (kNW * n + wu) * 1024);
    }
  };
  int bm, bn;
  auto start_tile = [&]() {
    tile_coords(t, ntm, ntn, bm, bn);
    const int m0 = bm * kBM;
    xa = reinterpret_cast<const char*>(p.x + (int64_t)m0 * p.x_st);
    wb = reinterpret_cast<const char*>(p.w + (int64_t)bn * nks * (kTileU * 8));
    const uint32_t last = (uint32_t)(p.M - 1 - m0);   // rows past M re-read row M-1
#pragma unroll
    for (int n = 0; n < kDI; ++n)
      xoff[n] = min(xrow[n], last) * (uint32_t)p.x_st * 2u + xchunk[n];
#pragma unroll
    for (int s = 0; s < kStages - 1; ++s) issue(s);
  };

  const int sw = (i32 >> 2) & 3;
  const int p0 = h ^ sw, p1 = (2 + h) ^ sw;
  const u32x4* sa0 = dsm + (wm * 128 + i32) * kRowU;
  const u32x4* sb0 = dsm + kTileU + (wn * 64 + i32) * kRowU;
  Frag f;
  auto rd = [&](int ks, int pp, int buf) {
    const int st = (ks % kStages) * kStageU + pp;
#pragma unroll
    for (int i = 0; i < kIM; ++i) f.a[buf][i] = __builtin_bit_cast(bf16x8, sa0[st + i * 32 * kRowU]);
#pragma unroll
    for (int j = 0; j < kJN; ++j) f.b[buf][j] = __builtin_bit_cast(bf16x8, sb0[st + j * 32 * kRowU]);
  };

  start_tile();
  for (;;) {
    const int kind = bn < p.nq ? kQ : bn < 2 * p.nq ? kK : bn < 4 * p.nq ? kV : kOG;
    const int m0 = bm * kBM, n0 = bn * kBN;
    if (kind == kV) {
      tile_main<false>(f, nks, issue, rd, p0, p1);
      // lane: column d = 32 wn + i32 of head bn - 2nq; v in j = 0, vg in j = 1;
      // register 4q+e: token m0 + 128 wm + 32 i + 8q + 4h + e
      const int head = bn - 2 * p.nq, d = wn * 32 + i32;
      const int nv = n0 + wn * 64 + i32;
      const float bv = p.bias[nv], bg = p.bias[nv + 32];
      // values are formed for every row (rows past M hold clamped-row data)
      // and only the stores are predicated
#pragma unroll
      for (int i = 0; i < kIM; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int m = m0 + wm * 128 + i * 32 + 8 * q + 4 * h;
          float o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float v = round_bf16(f.acc[i][0][4 * q + e] + bv);
            const float g = round_bf16(f.acc[i][1][4 * q + e] + bg);
            o[e] = round_bf16(v * round_bf16(sigmoidf_fast(g)));
          }
          const int b = m / p.T, tt = m - b * p.T;
          if (m < p.M)
            store4(p.vt + b * p.vt_sb + ((int64_t)head * 128 + d) * p.ldv + tt, o[0], o[1], o[2], o[3]);
        }
    } else {
      tile_main<true>(f, nks, issue, rd, p0, p1);
      // lane: token m0 + 128 wm + 32 i + i32; register 4q+e: column
      // n0 + 64 wn + 32 j + 8q + 4h + e
      const int cb = n0 + wn * 64 + 4 * h;                 // column of j = 0, q = 0
      floatx4 b0[4], b1[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        b0[q] = *reinterpret_cast<const floatx4*>(p.bias + cb + 8 * q);
        b1[q] = *reinterpret_cast<const floatx4*>(p.bias + cb + 8 * q + 32);
      }
#pragma unroll
      for (int i = 0; i < kIM; ++i) {
        const int m = m0 + wm * 128 + i * 32 + i32;
        const bool ok = m < p.M;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int c0 = cb + 8 * q;
          float x0[4], x1[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            x0[e] = round_bf16(f.acc[i][0][4 * q + e] + b0[q][e]);
            x1[e] = round_bf16(f.acc[i][1][4 * q + e] + b1[q][e]);
          }
          if (kind == kK) {
            // RoPE: out[d] = x[d] cos - x[d+64] sin, out[d+64] = x[d+64] cos + x[d] sin
            const int head = 2 * (bn - p.nq) + (wn >> 1);
            const int d = (wn & 1) * 32 + 8 * q + 4 * h;
            const int tt = m % p.T;
            float cs0[4], sn0[4], cs1[4], sn1[4];
            load4(p.cos + (int64_t)tt * p.cs_st + d, cs0);
            load4(p.sin + (int64_t)tt * p.cs_st + d, sn0);
            load4(p.cos + (int64_t)tt * p.cs_st + d + 64, cs1);
            load4(p.sin + (int64_t)tt * p.cs_st + d + 64, sn1);
            float y0[4], y1[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              y0[e] = round_bf16(round_bf16(x0[e] * cs0[e]) + round_bf16(-x1[e] * sn0[e]));
              y1[e] = round_bf16(round_bf16(x1[e] * cs1[e]) + round_bf16(x0[e] * sn1[e]));
            }
            uint16_t* ko = p.k_out + (int64_t)m * p.D + head * 128 + d;
            if (ok) {
              store4(ko, y0[0], y0[1], y0[2], y0[3]);
              store4(ko + 64, y1[0], y1[1], y1[2], y1[3]);
            }
          } else {
            uint16_t* o = kind == kQ ? p.q + (int64_t)m * p.q_st + c0 : p.og + (int64_t)m * p.og_st + (c0 - 4 * p.D);
            if (ok) {
              store4(o, x0[0], x0[1], x0[2], x0[3]);
              store4(o + 32, x1[0], x1[1], x1[2], x1[3]);
            }
          }
        }
      }
    }
    t += gx;
    if (t >= tend) break;
    asm volatile("s_barrier" ::: "memory");   // every wave has left the ring
    start_tile();
  }
}

// Zero keys [T, ldv) of every V^T row (the attention kernel reads whole 64-key tiles).
__global__ __launch_bounds__(256) void vt_pad_kernel(uint16_t* __restrict__ vt, int rows, int T, int ldv) {
  const int pad = ldv - T;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < (int64_t)rows * pad) {
    const int64_t r = i / pad;
    vt[r * ldv + T + (i - r * pad)] = 0;
  }
}

}  // namespace proj
}  // namespace gsa

// ---------------------------------------------------------------------------
// Host entry points
// ---------------------------------------------------------------------------
using namespace gsa_host;

namespace {
constexpr int kMaxDevices = 64;
bool g_proj_lds_set[kMaxDevices] = {};
int g_proj_cus[kMaxDevices] = {};

bool proj_shape_ok(int D, int H) { return H >= 2 && H <= 64 && D == 128 * H && D % 256 == 0; }
}  // namespace

extern "C" size_t gsa_proj_packed_bytes(int D, int H) {
  if (!proj_shape_ok(D, H)) return 0;
  return (size_t)5 * D * D * 2;
}

extern "C" int gsa_proj_pack(const void* w, int64_t w_st, const void* bias, int D, int H, int dtype,
                             void* w_packed, float* bias_packed, void* stream) {
  if (!w || !w_packed || !bias_packed) return GSA_ERR_NULL;
  if (dtype != GSA_DTYPE_BF16) return GSA_ERR_DTYPE;
  if (!proj_shape_ok(D, H) || w_st < D) return GSA_ERR_SHAPE;
  if (!aligned(w, 16) || w_st % 8 || !aligned(w_packed, 16) || !aligned(bias_packed, 4) ||
      (bias && !aligned(bias, 2)))
    return GSA_ERR_ALIGN;
  const int64_t units = (int64_t)5 * D * D / 8;
  hipLaunchKernelGGL(gsa::proj::pack_kernel, dim3((unsigned)((units + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<const uint16_t*>(w), w_st,
                     static_cast<const uint16_t*>(bias), D, static_cast<uint16_t*>(w_packed), bias_packed);
  return launch_status();
}

extern "C" int gsa_proj_fused(const void* x, int64_t x_st, int B, int T, int D, int H, int dtype,
                              const void* w_packed, const float* bias_packed,
                              const void* cos, const void* sin, int64_t cs_st,
                              void* q, int64_t q_st, void* og, int64_t og_st,
                              void* k_out, void* vt, int ldv, void* stream) {
  if (!x || !w_packed || !bias_packed || !cos || !sin || !q || !og || !k_out || !vt) return GSA_ERR_NULL;
  if (dtype != GSA_DTYPE_BF16) return GSA_ERR_DTYPE;
  if (!proj_shape_ok(D, H) || B < 1 || T < 1 || T % 64 != 0) return GSA_ERR_SHAPE;
  if (ldv < T || ldv % 64 != 0 || x_st < D || q_st < D || og_st < D || cs_st < 128) return GSA_ERR_SHAPE;
  const int64_t M = (int64_t)B * T;
  if (M > (1 << 26) || (int64_t)x_st * 2 * 256 > 0xffffffffLL) return GSA_ERR_SHAPE;
  if (!aligned(x, 16) || x_st % 8 || !aligned(w_packed, 16) || !aligned(bias_packed, 4) ||
      !aligned(q, 8) || q_st % 4 || !aligned(og, 8) || og_st % 4 || !aligned(k_out, 8) || !aligned(vt, 8) ||
      !aligned(cos, 8) || !aligned(sin, 8) || cs_st % 4)
    return GSA_ERR_ALIGN;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return GSA_ERR_SHAPE;
  if (!g_proj_lds_set[dev]) {   // more than the default 64 KiB of LDS per block
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(gsa::proj::proj_fused_kernel),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)gsa::proj::kLds);
    if (e != hipSuccess) return -static_cast<int>(e);
    int cus = 0;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (e != hipSuccess) return -static_cast<int>(e);
    g_proj_cus[dev] = cus;
    g_proj_lds_set[dev] = true;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (ldv > T) {
    const int rows = B * H * 128;
    const int64_t n = (int64_t)rows * (ldv - T);
    hipLaunchKernelGGL(gsa::proj::vt_pad_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                       static_cast<uint16_t*>(vt), rows, T, ldv);
    const int st = launch_status();
    if (st) return st;
  }
  const int nq = D / 256;
  const int64_t nt = ((M + 255) / 256) * 5 * nq;
  int grid = (g_proj_cus[dev] / 8) * 8;
  if (grid < 8) grid = 8;
  if ((int64_t)grid > (nt + 7) / 8 * 8) grid = (int)((nt + 7) / 8 * 8);
  gsa::proj::Args a{static_cast<const uint16_t*>(x), x_st, static_cast<const uint16_t*>(w_packed), bias_packed,
                    static_cast<const uint16_t*>(cos), static_cast<const uint16_t*>(sin), cs_st,
                    static_cast<uint16_t*>(q), q_st, static_cast<uint16_t*>(og), og_st,
                    static_cast<uint16_t*>(k_out), static_cast<uint16_t*>(vt), (int64_t)H * 128 * ldv, ldv,
                    (int)M, T, D, nq};
  hipLaunchKernelGGL(gsa::proj::proj_fused_kernel, dim3(grid), dim3(64 * gsa::proj::kNW), gsa::proj::kLds, s, a);
  return launch_status();
}
