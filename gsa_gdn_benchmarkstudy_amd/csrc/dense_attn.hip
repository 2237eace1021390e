// Block-dense sparse attention on gfx950 MFMA: every causal key tile is
// streamed once per query block and the exact top-k selection is
// applied as a bitmask, so masked-out keys get probability 0.  Same function
// as the gather kernel (softmax over each row's selected keys), different
// work: dense MFMA over the causal triangle instead of per-row gathers.
//
// Layouts: q, k [B,T,H,128]; v stored transposed, V^T [B,H,128,ldv] (written
// once by prologue_vt_kernel) so a key tile of V^T stages straight into LDS;
// selection bits [B,T,W] uint32, W = 2*ceil(Tkv/64): bit j of row t set iff
// key j is selected and valid for query t.
//
// Per block: one head, 256 query rows (8 waves of 32 rows), 64-key tiles in
// LDS.  With
// v_mfma_f32_32x32x16_bf16 both products are computed transposed,
//   S^T = K Q^T    (A = K tile from LDS, B = this wave's q, in registers)
//   O^T = V^T P^T  (A = V^T tile from LDS, B = P in registers)
// so in both outputs lane l holds column l%32 = one query row: a query's
// softmax state lives in its two lanes (l and l^32) and P never moves between
// lanes.  Accumulator r of lane l is row 8*(r/4) + 4*(l/32) + r%4 of the
// 32x32 block: head dims of O^T; the rows of S^T are keys in the permuted
// order described at the dense kernel.
#include "gsa_common.h"

namespace gsa {

// Waves per dense-attention block (32 query rows each).  The mask-operand
// layout pads its 32-row groups to whole blocks.
constexpr int kDenseWaves = 8;
constexpr int kDK = 64;          // keys per tile
constexpr int kKS = 128 + 8;     // LDS row stride of prologue_vt's staging tile (elements)

// ---------------------------------------------------------------------------
// Producer with transposed V: k_out = RoPE(k) [B,T,H,128], vt = (v*sigmoid(vg))^T
// [B,H,128,ldv]; keys in [T, ldv) of vt are written as zeros.  One block per
// (b, h, 64-key tile).
// ---------------------------------------------------------------------------
struct ProVtArgs {
  const uint16_t* k; int64_t k_sb, k_st;
  const uint16_t* v; int64_t v_sb, v_st;
  const uint16_t* vg; int64_t g_sb, g_st;
  const uint16_t* cos; const uint16_t* sin; int64_t cs_st;
  uint16_t* k_out;
  uint16_t* vt;
  int T, H, ldv, ntiles;
};

// Block `blk` of the producer (one (b, h, 64-key tile)); sV: kDK * kKS elements of LDS.
__device__ __forceinline__ void prologue_vt_block(const ProVtArgs& p, int blk, uint16_t* sV) {
  // heads fastest: the blocks that run side by side read one key tile's
  // rows of every head (4 KiB of contiguous k, v and vg per key)
  const int h = blk % p.H;
  const int kt = (blk / p.H) % p.ntiles;
  const int b = blk / (p.H * p.ntiles);
  const int j0 = kt * kDK;
  const int tid = threadIdx.x, li = tid & 15;
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int item = it * 256 + tid;
    const int key = item >> 4, c = item & 15;   // c == li: one key per 16-lane row
    const int j = j0 + key;
    u32x4 packed = {0u, 0u, 0u, 0u};
    if (j < p.T) {
      if (p.k) {
        float x[8], cs[8], sn[8];
        load8(p.k + b * p.k_sb + (int64_t)j * p.k_st + h * 128 + c * 8, x);
        load8(p.cos + (int64_t)j * p.cs_st + c * 8, cs);
        load8(p.sin + (int64_t)j * p.cs_st + c * 8, sn);
        rope8<uint16_t>(x, cs, sn, li);
        store8(p.k_out + (((int64_t)b * p.T + j) * p.H + h) * 128 + c * 8, x);
      }
      float vv[8], gg[8];
      load8(p.v + b * p.v_sb + (int64_t)j * p.v_st + h * 128 + c * 8, vv);
      load8(p.vg + b * p.g_sb + (int64_t)j * p.g_st + h * 128 + c * 8, gg);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float a = round_bf16(vv[2 * i] * round_bf16(sigmoidf_fast(gg[2 * i])));
        const float z = round_bf16(vv[2 * i + 1] * round_bf16(sigmoidf_fast(gg[2 * i + 1])));
        packed[i] = pack_bf16(a, z);
      }
    }
    *reinterpret_cast<u32x4*>(sV + key * kKS + c * 8) = packed;
  }
  __syncthreads();
  uint16_t* vtb = p.vt + ((int64_t)b * p.H + h) * 128 * p.ldv;
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int item = it * 256 + tid;
    const int d = item >> 3, c8 = item & 7;     // 128 rows x 8 chunks of 8 keys
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = (uint32_t)sV[(8 * c8 + 2 * i) * kKS + d] | ((uint32_t)sV[(8 * c8 + 2 * i + 1) * kKS + d] << 16);
    *reinterpret_cast<u32x4*>(vtb + (int64_t)d * p.ldv + j0 + 8 * c8) = w;
  }
}

__global__ __launch_bounds__(256) void prologue_vt_kernel(ProVtArgs p) {
  __shared__ __align__(16) uint16_t sV[kDK * kKS];
  prologue_vt_block(p, blockIdx.x, sV);
}

// ---------------------------------------------------------------------------
// Selection bitmask from (indices, count, mask): one block per row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void selection_mask_kernel(
    const int32_t* __restrict__ idx, int64_t i_sb, int64_t i_st, int k_sel,
    const int32_t* __restrict__ count, const uint8_t* __restrict__ mask, int T, int Tkv, int W,
    uint32_t* __restrict__ bits, int64_t b_sb, int64_t b_st) {
  extern __shared__ uint32_t sw[];
  const int row = blockIdx.x;
  const int b = row / T, t = row % T;
  for (int i = threadIdx.x; i < W; i += 256) sw[i] = 0u;
  __syncthreads();
  int n = k_sel;
  if (count) n = min(n, count[row]);
  const int64_t base = b * i_sb + (int64_t)t * i_st;
  for (int m = threadIdx.x; m < n; m += 256) {
    if (mask == nullptr || mask[base + m] != 0) {
      const int j = min(max(idx[base + m], 0), Tkv - 1);
      atomicOr(&sw[j >> 5], 1u << (j & 31));
    }
  }
  __syncthreads();
  uint32_t* brow = bits + b * b_sb + (int64_t)t * b_st;
  for (int i = threadIdx.x; i < W; i += 256) brow[i] = sw[i];
}

// ---------------------------------------------------------------------------
// Selection bitmask -> the dense kernel's mask operands.
// The dense kernel applies the selection inside its S^T accumulators: each
// 32-key half starts with one v_mfma_scale_f32_32x32x64_f8f6f4 on e2m1 (fp4)
// operands, an identity A (lane (h, m) of half c holds 1.0 at the k position
// of the key that MFMA row m holds, when h == c) times a mask B scaled by
// 2^kMaskExp, so the accumulator starts at +0 for a selected key and at
// -6 * 2^kMaskExp for any other; the bf16 products then add onto that.
// For 32-row group g (rows 32g + n), 64-key tile kt and lane l = 32h + n of
// the wave that owns the group, mop[b][g][kt][l] (16 bytes) is that B operand:
// nibble i (bits 4i .. 4i+3 of the 128-bit value) is 0x0 (+0.0) if row 32g+n
// selects key 64kt + 32h + i, else 0xF (-6.0).  One 1 KiB record per
// (group, tile), in the order the kernel's wave stages it into LDS.
// One thread per (row, 4 consecutive tiles): it reads the row's 32 bytes of
// selection words and writes lanes n and 32 + n of each tile's record.
// ---------------------------------------------------------------------------
constexpr int kLmTiles = 4;
constexpr int kMaskExp = 120;          // unselected keys start at -6 * 2^120 (about -8e36)
constexpr float kNoKey = -1e36f;       // a tile row max below this: no selected key in the tile

struct LaneMaskArgs {
  const uint32_t* bits; int64_t b_sb, b_st;
  int T, G, NT, nunits;   // unit = (batch, 32-row group, kLmTiles tiles): 32 threads
  int block_rows;         // causal: query rows per attention block (tiles past a block's last row are skipped); else 0
  u32x4* lm;
};

// Bit i of an 8-bit value moved to bit 4i.
__device__ __forceinline__ uint32_t spread_nibbles(uint32_t byte) {
  uint32_t t = (byte | (byte << 12)) & 0x000F000Fu;
  t = (t | (t << 6)) & 0x03030303u;
  return (t | (t << 3)) & 0x11111111u;
}
// 32 selection bits -> 32 e2m1 nibbles: 0x0 where the bit is set, 0xF where not.
__device__ __forceinline__ u32x4 mask_nibbles(uint32_t word) {
  const uint32_t un = ~word;
  u32x4 r;
#pragma unroll
  for (int j = 0; j < 4; ++j) r[j] = spread_nibbles((un >> (8 * j)) & 0xffu) * 15u;
  return r;
}

// Block `blk` of the mask-operand pass: its 256 threads take units 8*blk .. 8*blk+7.
__device__ __forceinline__ void lane_mask_block(const LaneMaskArgs& a, int blk) {
  const int gt = blk * 256 + (int)threadIdx.x;
  const int unit = gt >> 5, n = gt & 31;
  if (unit >= a.nunits) return;
  const int nq = (a.NT + kLmTiles - 1) / kLmTiles;
  const int kq = unit % nq, bg = unit / nq;
  const int g = bg % a.G, b = bg / a.G;
  const int row = 32 * g + n;
  const int kt0 = kq * kLmTiles;
  // Tiles the attention reads for this group: all of them, or (causal) those
  // up to the last row of the group's attention block, as its block does.
  int nt = a.NT;
  if (a.block_rows) nt = min(a.NT, ((32 * g) / a.block_rows + 1) * a.block_rows / kDK);
  if (kt0 >= nt) return;
  const uint64_t* src =
      reinterpret_cast<const uint64_t*>(a.bits + b * a.b_sb + (int64_t)min(row, a.T - 1) * a.b_st) + kt0;
  uint64_t words[kLmTiles];
#pragma unroll
  for (int u = 0; u < kLmTiles; ++u) words[u] = (row < a.T && kt0 + u < nt) ? src[u] : 0ull;
#pragma unroll
  for (int u = 0; u < kLmTiles; ++u) {
    if (kt0 + u >= nt) break;
    u32x4* dst = a.lm + ((int64_t)bg * a.NT + kt0 + u) * 64;
    dst[n] = mask_nibbles((uint32_t)words[u]);
    dst[32 + n] = mask_nibbles((uint32_t)(words[u] >> 32));
  }
}

__global__ __launch_bounds__(256) void lane_mask_kernel(LaneMaskArgs a) { lane_mask_block(a, blockIdx.x); }

// The producer and the lane-mask pass in one launch, their blocks interleaved
// evenly over the grid so that both kinds run side by side: block b is a
// lane-mask block iff c(b+1) > c(b), c(b) = floor(b * n_lm / (n_pro + n_lm))
// (the number of lane-mask blocks before b), with lane-mask index c(b) and
// producer index b - c(b).
__global__ __launch_bounds__(256) void prologue_vt_lane_mask_kernel(ProVtArgs p, LaneMaskArgs l, int n_pro,
                                                                    int n_lm) {
  __shared__ __align__(16) uint16_t sV[kDK * kKS];
  const int64_t total = (int64_t)n_pro + n_lm, b = blockIdx.x;
  const int c0 = (int)(b * n_lm / total), c1 = (int)((b + 1) * n_lm / total);
  if (c1 > c0) lane_mask_block(l, c0);
  else prologue_vt_block(p, (int)(b - c0), sV);
}

// ---------------------------------------------------------------------------
// Dense masked attention (bf16)
//
// Block: 8 waves = 256 query rows of one head (wave w: rows 32w .. 32w+31),
// two waves per SIMD.  K and V^T tiles and each wave's mask operands reach
// LDS by direct
// global->LDS loads (16 B per lane; one instruction fills 1 KiB,
// lane-linear), each through a pair of slots, K and V^T in padded layouts
// (unit = 16 B = 8 bf16):
//   K   tile: 64 keys x 17 units, unit 16 of a key is padding
//   V^T tile: 128 rows x 9 units (64 keys), unit 8 of a row is padding
//   mask:     8 waves x 64 units (each lane's 16-byte B operand)
// The odd row strides make every MFMA operand read conflict-free (16 lanes
// reading one unit of 16 different rows hit 16 different bank groups), and
// each operand read is one base register plus an immediate offset.  Padding
// units receive a harmless duplicate load.
// Key order: in the S^T product of a 32-key half, MFMA row rho holds key
// pi(rho), pi swapping bits 2 and 3 of rho, so accumulator r of lane (h, i)
// holds key 16(r/8) + 8h + r%8.  A lane's 8 P values of each 16-key k-step
// are then contiguous keys, and its V^T operand is one 16-byte read.
// Masking: each half's S^T accumulators start from the fp4 mask product
// (+0 selected, about -8e36 not selected; lane_mask_block), so the softmax
// takes its row max and exponentials straight from the accumulators: a
// key that is not selected gets p = 2^(-huge) = 0, and the scores of the
// selected keys are the bf16 products alone, bit for bit.  No mask word
// passes through scalar registers and the loop issues no scalar load.
//
// Tiles are pipelined: S^T of tile t+1 is computed, one 32-key half at a
// time, while tile t's row maxima are taken, then the tile's one
// online-softmax decision with the lazy reference (below), then O^T +=
// V^T(t) P^T(t) half by half, so MFMA and VALU work of one wave overlap.
// ---------------------------------------------------------------------------
struct DenseArgs {
  const uint16_t* q; int64_t q_sb, q_st;
  const uint16_t* k; int64_t k_sb, k_st;
  const uint16_t* vt; int64_t vt_sb, vt_sh; int ldv;
  int G, NT;                              // mask operands [B][G][NT][64] u32x4 (kernel argument)
  const uint16_t* og; int64_t o_sb, o_st;
  const uint16_t* cos; const uint16_t* sin; int64_t cs_st;
  uint16_t* out; int64_t out_sb, out_st;
  int B, T, Tkv, H, nqb;
  float scale_l2;
  int flags;
};

constexpr int kDenseCausal = 1 << 8;   // internal flag: skip key tiles after the block's last row
constexpr float kLazy = 8.f;           // log2 headroom of the lazy softmax reference
constexpr int kKRow = 17, kVRow = 9;   // padded row lengths in 16-byte units
constexpr int kKU = kDK * kKRow;       // 1088 units: K tile
constexpr int kVU = 128 * kVRow;       // 1152 units: V^T tile
constexpr int kDmaK = kKU / 64;        // 17 load instructions fill a K tile
constexpr int kDmaV = kVU / 64;        // 18 fill a V^T tile
constexpr int kMBase = 2 * (kKU + kVU);   // units: two K slots, two V^T slots, then the two mask slots
constexpr int kXBase = kMBase + 2 * 64 * kDenseWaves;   // units: the waves' 8 KiB staging tiles
// LDS of a block: the K and V^T slot pairs, two mask slots of 8 KiB, and one
// 8 KiB staging tile per wave (q, the RoPE tables and the output gate on
// the way in, the output on the way out).
constexpr size_t kDenseLds = (size_t)(kXBase + 512 * kDenseWaves) * 16;

// Staging tile: 32 rows x 256 bytes (16 chunks of 16 bytes); chunk c of row
// r sits at chunk slot c ^ (r & 15), so that a row load (4 rows x 256 bytes
// per instruction, lane-linear) and an operand read (one chunk of 32 rows)
// are both conflict-free.  Unit offset of (row, chunk) within the tile:
__device__ __forceinline__ int xs_unit(int row, int chunk) { return row * 16 + (chunk ^ (row & 15)); }

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef int intx8 __attribute__((ext_vector_type(8)));

// Value of lane l^32 combined with the own value: permlane32_swap of (v, v)
// leaves {v[l], v[l^32]} in the two results on every lane.  max_halves takes
// values that are never NaN (maxima seeded with -inf), so a compare-select
// is enough (fmaxf would first quiet both operands).
__device__ __forceinline__ float max_halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  const float a = __uint_as_float(r[0]), b = __uint_as_float(r[1]);
  return a > b ? a : b;
}
__device__ __forceinline__ float sum_halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// 32-bit LDS address of a shared-memory pointer.
__device__ __forceinline__ uint32_t lds_addr(const void* ptr) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)ptr;
}

// Direct global -> LDS load: every lane's 16 bytes at base + voff land at
// lds + 16 * lane (base and lds uniform).  Issued as inline asm so that the
// compiler's own bookkeeping does not make each LDS read wait for every such
// load in flight; completion is awaited explicitly (vmcnt) before the
// barrier that publishes a tile.  m0 holds the LDS address; nothing else in
// this kernel uses m0.  An LDS DMA reads m0 one wait state after the SALU
// write at the earliest (the s_nop; the compiler pads its own LDS DMA the
// same way on gfx950).
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void load_lds16(const void* base, uint32_t voff, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// s_waitcnt immediate (gfx9 encoding): vmcnt(0), expcnt and lgkmcnt not waited
constexpr int kWaitVmcnt0 = (0x7 << 4) | (0xf << 8);

__device__ __forceinline__ int swap_bits23(int i) { return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1); }

template <int N> struct Int { static constexpr int value = N; };

// Pipeline of one block (8 waves = 256 query rows of one head), tile t = 64
// keys.  K tiles, V^T tiles and mask operands stream through separate pairs
// of LDS slots (tile t in slot t&1).  Iteration t, after one barrier:
//   loads  K(t+2) and its mask operands into K / mask slot t&1 (S(t) was
//          computed last iteration) and V^T(t+1) into V slot (t+1)&1 (PV(t-1)
//          is done);
//   MFMA   S^T(t+1) from K slot (t+1)&1, interleaved with the row maxima of
//          S(t) (VALU), then O^T += V^T(t) P^T(t) from V slot t&1.
// So the S product of the next tile overlaps the softmax of this one, within
// the wave, at the cost of a second S accumulator pair (64 VGPRs).  Every
// load is issued one iteration before the barrier that publishes it; the
// loop is unrolled by two so that slot offsets are constants.
__global__ __launch_bounds__(64 * kDenseWaves, 1) void dense_attn_kernel(DenseArgs p, const u32x4* __restrict__ lm) {
  extern __shared__ __align__(16) u32x4 dsm[];   // K slots 0, 1 (kKU units each), V^T slots 0, 1 (kVU), mask slots 0, 1 (512)
  constexpr int kDW = kDenseWaves;                // waves per block
  constexpr int kDQ = 32 * kDW;                   // query rows per block
  constexpr int kDmaKW = (kDmaK + kDW - 1) / kDW;   // K instructions per wave (wave w: i = kDW*n + w < 17)
  constexpr int kDmaVW = (kDmaV + kDW - 1) / kDW;   // V^T instructions per wave
  constexpr int kMSlot = 64 * kDW;                // units of one mask slot

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wu = __builtin_amdgcn_readfirstlane(w);
  const int i32 = lane & 31, h = lane >> 5;
  // The wave's 32-row group within the block: waves w and w+4 (one SIMD)
  // take groups w and 7-w, so that in a causal block each SIMD's two waves
  // skip the same number of key tiles past their rows (3 + 0, 3 + 0, 2 + 1,
  // 2 + 1).  Loads into LDS and the staging tile stay indexed by the wave.
  const int gw = wu < 4 ? wu : 11 - wu;
  // Block order: batch by batch (the blocks in flight then share one
  // sequence's K and V^T, which stays in the last-level cache), within a
  // sequence the heaviest query blocks first, heads fastest.
  const int per_b = p.nqb * p.H;
  const int b = (int)(blockIdx.x / per_b);
  const int r2 = (int)(blockIdx.x % per_b);
  const int qb = p.nqb - 1 - r2 / p.H;
  const int hd = r2 % p.H;
  const int q0 = qb * kDQ;

  const int last_key = (p.flags & kDenseCausal) ? min(p.Tkv - 1, q0 + kDQ - 1) : p.Tkv - 1;
  const int nkt = last_key / kDK + 1;
  const char* kbase = reinterpret_cast<const char*>(p.k + b * p.k_sb + hd * 128);
  const char* vtb = reinterpret_cast<const char*>(p.vt + b * p.vt_sb + hd * p.vt_sh);
  const int64_t kstep = (int64_t)kDK * p.k_st * 2;             // bytes from one K tile to the next
  const uint32_t lds0 = __builtin_amdgcn_readfirstlane(lds_addr(dsm));

  // ---- tile loads: wave w issues K instructions i = kDW*n + w < 17 and V^T
  // instructions i = kDW*n + w < 18.  K instruction i fills K units
  // 64i .. 64i+63 (key u/17, unit u%17), V^T instruction i units 64i .. (row
  // u/9, unit u%9).  koff/voff = this lane's source byte offset from the
  // tile's K or V^T base (32-bit: the host bounds k_st and ldv); koff_last
  // for the last tile, whose keys past Tkv-1 re-read key Tkv-1.  Each wave
  // also loads its own group's 1 KiB of mask operands per tile.
  const int nkw = (kDmaK - 1 - wu) / kDW + 1;    // this wave's K instructions (uniform)
  const int nvw = (kDmaV - 1 - wu) / kDW + 1;    // and V^T instructions
  uint32_t koff[kDmaKW], koff_last[kDmaKW], voff[kDmaVW];
  {
    const uint32_t kst2 = (uint32_t)p.k_st * 2u, ldv2 = (uint32_t)p.ldv * 2u;
    const int kmax_last = min(kDK - 1, p.Tkv - 1 - (nkt - 1) * kDK);
    auto k_off = [&](int i, int kmax) {
      const int u = i * 64 + lane, key = u / kKRow, c = u - key * kKRow;
      return (uint32_t)min(key, kmax) * kst2 + (uint32_t)min(c, 15) * 16u;
    };
#pragma unroll
    for (int n = 0; n < kDmaKW; ++n) {
      const int i = min(kDW * n + wu, kDmaK - 1);
      koff[n] = k_off(i, kDK - 1);
      koff_last[n] = k_off(i, kmax_last);
    }
#pragma unroll
    for (int n = 0; n < kDmaVW; ++n) {
      const int u = min(kDW * n + wu, kDmaV - 1) * 64 + lane, d = u / kVRow, c = u - d * kVRow;
      voff[n] = (uint32_t)d * ldv2 + (uint32_t)min(c, 7) * 16u;
    }
  }
  const uint32_t kdst = lds0 + (uint32_t)wu * 1024u;                      // + slot * kKU * 16 + n * kDW KiB
  const uint32_t vdst = lds0 + (uint32_t)(2 * kKU * 16) + (uint32_t)wu * 1024u;
  const uint32_t mdst = lds0 + (uint32_t)(kMBase * 16) + (uint32_t)wu * 1024u;   // + slot * kDW KiB
  // this wave's mask operands: group kDW*qb + w, 1 KiB per tile
  const char* mbase = reinterpret_cast<const char*>(lm + ((int64_t)b * p.G + kDW * qb + gw) * p.NT * 64);
  const uint32_t moff = (uint32_t)lane * 16u;
  auto issue_k = [&](const char* src, int slot, bool last) {   // one K tile into K slot `slot`
#pragma unroll
    for (int n = 0; n < kDmaKW; ++n)
      if (n + 1 < kDmaKW || n < nkw)
        load_lds16(src, last ? koff_last[n] : koff[n], kdst + (uint32_t)(slot * kKU * 16 + n * kDW * 1024));
  };
  auto issue_v = [&](const char* src, int slot) {              // one V^T tile into V slot `slot`
#pragma unroll
    for (int n = 0; n < kDmaVW; ++n)
      if (n + 1 < kDmaVW || n < nvw)
        load_lds16(src, voff[n], vdst + (uint32_t)(slot * kVU * 16 + n * kDW * 1024));
  };
  auto issue_m = [&](int kt, int slot) {                       // tile kt's mask operands into mask slot `slot`
    load_lds16(mbase + (int64_t)kt * 1024, moff, mdst + (uint32_t)(slot * kDW * 1024));
  };
  // ---- the wave's staging tile (rows q0 + 32w .. +31, clamped to T-1; 256
  // bytes each at a column offset): 8 loads of 4 rows x 256 bytes, each
  // lane's 16 bytes placed by the tile's chunk swizzle.  Loading whole rows
  // per instruction keeps every load to 8 cache lines; a lane-per-row load
  // of the same data touches 32 lines per instruction, and a block's
  // prologue then waited several microseconds for its q, cos and sin.
  const int rbase = min(q0 + 32 * gw, p.T - 1);
  const uint32_t xdst = lds0 + (uint32_t)((kXBase + wu * 512) * 16);
  const u32x4* xt = dsm + kXBase + wu * 512;
  auto stage = [&](const uint16_t* base, int64_t row_st) {   // base: element (rbase, column offset)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int r = 4 * j + (lane >> 4);
      const uint32_t roff = (uint32_t)(min(q0 + 32 * gw + r, p.T - 1) - rbase);
      load_lds16(base, roff * (uint32_t)(row_st * 2) + (uint32_t)(((lane & 15) ^ (r & 15)) * 16),
                 xdst + (uint32_t)(j * 1024));
    }
  };

  // ---- q: B operand of S^T; lane supplies d = 16s + 8h .. +7 of its row ----
  stage(p.q + b * p.q_sb + (int64_t)rbase * p.q_st + hd * 128, p.q_st);
  // prologue loads: K(0), K(1), V(0) and the mask operands of the same
  // tiles, issued after q's so that q does not wait behind them: every wave
  // issues at least 5 of them (2 K, 1 mask, 2 V^T), so vmcnt(5) leaves only
  // tile loads in flight
  issue_k(kbase, 0, nkt == 1);
  issue_m(0, 0);
  if (nkt > 1) {
    issue_k(kbase + kstep, 1, nkt == 2);
    issue_m(1, 1);
  }
  issue_v(vtb, 0);
  asm volatile("s_waitcnt vmcnt(5)" ::: "memory");   // this wave's q rows have landed
  u32x4 qraw[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) qraw[s] = xt[xs_unit(i32, 2 * s + h)];
  if (p.flags & GSA_ATTN_ROPE_Q) {
    // the cos and sin rows through the same tile, after the q reads returned:
    // one round for a packed table (row: cos[0:64] then sin[0:64]; entries d
    // and d+64 are equal), else cos, then sin
    u32x4 craw[8], sraw[8];
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    stage(p.cos + (int64_t)rbase * p.cs_st, p.cs_st);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (p.flags & GSA_ATTN_ROPE_HALVES) {
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        craw[s] = craw[s + 4] = xt[xs_unit(i32, 2 * s + h)];
        sraw[s] = sraw[s + 4] = xt[xs_unit(i32, 8 + 2 * s + h)];
      }
    } else {
#pragma unroll
      for (int s = 0; s < 8; ++s) craw[s] = xt[xs_unit(i32, 2 * s + h)];
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      stage(p.sin + (int64_t)rbase * p.cs_st, p.cs_st);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
      for (int s = 0; s < 8; ++s) sraw[s] = xt[xs_unit(i32, 2 * s + h)];
    }
    auto unpack8 = [](const u32x4& v, float (&x)[8]) {
#pragma unroll
      for (int i = 0; i < 4; ++i) { x[2 * i] = bf16lo(v[i]); x[2 * i + 1] = bf16hi(v[i]); }
    };
    // rotate_half partner of d (d < 64: -x[d+64]; else x[d-64]) is register s^4
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      float c0[8], s0[8], c1[8], s1[8];
      unpack8(craw[s], c0);
      unpack8(sraw[s], s0);
      unpack8(craw[s + 4], c1);
      unpack8(sraw[s + 4], s1);
      float lo[8], hi[8], ylo[8], yhi[8];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        lo[2 * j] = bf16lo(qraw[s][j]); lo[2 * j + 1] = bf16hi(qraw[s][j]);
        hi[2 * j] = bf16lo(qraw[s + 4][j]); hi[2 * j + 1] = bf16hi(qraw[s + 4][j]);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        ylo[j] = round_bf16(round_bf16(lo[j] * c0[j]) + round_bf16(-hi[j] * s0[j]));
        yhi[j] = round_bf16(round_bf16(hi[j] * c1[j]) + round_bf16(lo[j] * s1[j]));
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        qraw[s][j] = pack_bf16(ylo[2 * j], ylo[2 * j + 1]);
        qraw[s + 4][j] = pack_bf16(yhi[2 * j], yhi[2 * j + 1]);
      }
    }
  }
  bf16x8 qop[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) qop[s] = __builtin_bit_cast(bf16x8, qraw[s]);

  // Identity A operands of the mask products (e2m1 1.0 = 0x2): half c, lane
  // (h, m): the k position of key pi(m) of the half -- position pi(m) of the
  // lane's 32 -- when h == c, nothing otherwise.  Only the first four
  // registers of an fp4 operand are read.
  intx8 ident[2];
  {
    const int pos = swap_bits23(i32);
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int j = 0; j < 8; ++j) ident[c][j] = (h == c && j == (pos >> 3)) ? (2 << (4 * (pos & 7))) : 0;
  }

  floatx16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;
  // softmax state of the lane's row: reference m (log2 domain), m + kLazy,
  // -m (0 while m = -inf), and the running sum l
  float m = -__builtin_inff(), mlz = -__builtin_inff(), nm = 0.f, l = 0.f;
  const bf16x2 ones2 = __builtin_bit_cast(bf16x2, 0x3f803f80u);   // (1, 1)

  // operand read offsets (units within a slot): K row of MFMA row i32, V^T row i32, own mask operand
  const int kread = swap_bits23(i32) * kKRow + h;
  const int vread = 2 * kKU + i32 * kVRow + h;
  const int mread = kMBase + wu * 64 + lane;

  // the mask operands of the tile in mask slot ms (B operand, fp4: first four registers)
  auto mask_op = [&](int ms) {
    const u32x4 v = dsm[mread + ms * kMSlot];
    return intx8{(int)v[0], (int)v[1], (int)v[2], (int)v[3], 0, 0, 0, 0};
  };
  // S^T of one 32-key half of the tile in K slot ks, starting from its mask product
  auto s_half = [&](int ks, int c, const intx8& mop) {
    const u32x4* sK = dsm + ks * kKU + kread;
    bf16x8 f[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) f[s] = __builtin_bit_cast(bf16x8, sK[32 * c * kKRow + 2 * s]);
    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ident[c], mop, acc, 4, 4, 0, 127, 0, 127 + kMaskExp);
#pragma unroll
    for (int s = 0; s < 8; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[s], qop[s], acc, 0, 0, 0);
    return acc;
  };
  // Masked online softmax, one step per 64-key tile: p = 2^(s*scale*log2e -
  // m) against a per-row reference m that only moves when the tile's row max
  // over its selected keys exceeds it by more than kLazy (p <= 2^kLazy; out =
  // O / l does not depend on m).  max_half takes a half's maximum straight
  // from its accumulators (a key that is not selected sits near -8e36 there);
  // both halves are taken before the tile's one reference decision, so the S^T
  // MFMAs of the next tile share that stretch of code.  A maximum below kNoKey
  // means no selected key.  A move is rare: its bookkeeping -- alpha =
  // 2^(m_old - m_new), O and l times alpha, the new m, m + kLazy and -m --
  // runs in a branch the wave takes only when one of its rows moves.
  // exp_half turns a half's scores into P (two B operands of O^T) and adds
  // the bf16 values that the PV product uses to l, one dot2 per pair.
  auto max_half = [&](const floatx16& acc) -> float {
    float mx = -__builtin_inff();
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, acc[r]);
    return mx;                                      // never NaN: the max is seeded with -inf
  };
  auto exp_half = [&](const floatx16& acc, uint32_t (&pk)[2][4]) {
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[r], p.scale_l2, nm));
      const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[r + 1], p.scale_l2, nm));
      const uint32_t w = pack_bf16(p0, p1);
      pk[r >> 3][(r & 7) >> 1] = w;
      l = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), ones2, l, false);
    }
  };
  auto rescale = [&](float alpha) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[dt][r] *= alpha;
  };
  auto pv_half = [&](int vs, int c, const uint32_t (&pk)[2][4]) {
    const u32x4* sV = dsm + vs * kVU + vread;
    bf16x8 f[2][4];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
        f[ks][dt] = __builtin_bit_cast(bf16x8, sV[32 * dt * kVRow + 4 * c + 2 * ks]);
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const bf16x8 pb = __builtin_bit_cast(bf16x8, u32x4{pk[ks][0], pk[ks][1], pk[ks][2], pk[ks][3]});
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[ks][dt], pb, o[dt], 0, 0, 0);
    }
  };

  // Prologue loads and the q loads have landed.  The wait is the compiler's
  // own intrinsic, so it knows that none of its loads is still in flight and
  // puts no vmcnt wait into the loop, where the counter also counts the tile
  // loads and any such wait would drain them.
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();
  // The second wave of each SIMD issues first whenever both are ready: the
  // two waves leave each barrier together, and an even arbitration keeps
  // them in step (both in their MFMA stretches, then both in their softmax
  // VALU stretches); with one of them ahead, one wave's softmax runs beside
  // the other's products.  1-1.5 % faster at T = 16384 than equal priority.
  if (wu >= 4) __builtin_amdgcn_s_setprio(2);
  const char* vsrc = vtb + kDK * 2;                  // V^T tile kt+1
  // Tile kt once both halves' maxima are taken: the softmax decision, P and
  // O^T += V^T(kt) P^T(kt) from V slot vs.
  auto softmax_pv = [&](int vs, float mx0, float mx1, const floatx16& s0, const floatx16& s1) {
    float mx = max_halves(mx1 > mx0 ? mx1 : mx0);
    mx = mx > kNoKey ? mx * p.scale_l2 : -__builtin_inff();
    // mx > m + kLazy; while m = -inf: any selected key
    if (ballot64(mx > mlz)) {
      const bool bump = mx > mlz;
      const float alpha = bump ? __builtin_amdgcn_exp2f(m - mx) : 1.f;   // m = -inf -> 0
      rescale(alpha);
      l *= alpha;
      m = bump ? mx : m;
      mlz = m + kLazy;
      nm = m == -__builtin_inff() ? 0.f : -m;
    }
    uint32_t pk0[2][4], pk1[2][4];
    exp_half(s0, pk0);
    pv_half(vs, 0, pk0);
    exp_half(s1, pk1);
    pv_half(vs, 1, pk1);
  };

  // S^T of tile kt in sc[kt & 1]: with the loop unrolled by two, each
  // iteration writes the other pair, so no accumulator is copied
  // key tiles this wave computes: up to its last row when causal (uniform)
  const int nkw_t = (p.flags & kDenseCausal) ? min(nkt, min(p.Tkv - 1, q0 + 32 * gw + 31) / kDK + 1) : nkt;
  floatx16 sc[2][2];
  {
    const intx8 mop = mask_op(0);
    sc[0][0] = s_half(0, 0, mop);
    sc[0][1] = s_half(0, 1, mop);                 // S^T of tile 0
  }
  const char* ksrc = kbase + 2 * kstep;            // K tile kt+2
  // Iteration kt, first half: this wave's loads of K(kt+1), its mask
  // operands and V^T(kt) (issued last iteration) are done and its LDS reads
  // have returned; the barrier publishes every wave's loads and frees K and
  // mask slot P = kt & 1 and V slot 1-P for the next loads.
  auto sync_issue = [&](int kt, int P) {
    asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (kt + 2 < nkt) {
      issue_k(ksrc, P, kt + 3 == nkt);
      issue_m(kt + 2, P);
    }
    if (kt + 1 < nkt) issue_v(vsrc, 1 - P);
    ksrc += kstep;
    vsrc += kDK * 2;
    // the output-gate rows into the staging tile (free since the q and RoPE
    // reads before the first barrier), awaited at the next barrier
    if (kt == 0 && (p.flags & GSA_ATTN_OUT_GATE)) stage(p.og + b * p.o_sb + (int64_t)rbase * p.o_st + hd * 128, p.o_st);
  };
  // One iteration: S^T(kt+1) (stale on the wave's last tile, unused) ||
  // softmax(kt), then PV(kt).
  auto step = [&](int kt, auto par) {
    constexpr int P = decltype(par)::value;
    sync_issue(kt, P);
    const intx8 mop = mask_op(1 - P);
    sc[1 - P][0] = s_half(1 - P, 0, mop);
    const float mx0 = max_half(sc[P][0]);
    sc[1 - P][1] = s_half(1 - P, 1, mop);
    const float mx1 = max_half(sc[P][1]);
    softmax_pv(P, mx0, mx1, sc[P][0], sc[P][1]);
  };
  // Tiles 0 .. nkw_t-1 with their products (unrolled by two so that slot
  // offsets are constants), then the block's remaining tiles -- past this
  // wave's last row when causal: they hold no selected key of its rows, so
  // their products would add exact zeros -- with the loads and barriers only.
  int t = 0;
  for (; t + 1 < nkw_t; t += 2) {
    step(t, Int<0>{});
    step(t + 1, Int<1>{});
  }
  if (t < nkw_t) {
    step(t, Int<0>{});
    ++t;
  }
  for (; t < nkt; ++t) sync_issue(t, t & 1);

  // ---- epilogue: normalise, bf16, optional output gate ----
  l = sum_halves(l);
  // O / l as O * (1/l): one division per row instead of one per element
  // (the product is within 1.5 fp32 ulp of the quotient before the bf16
  // rounding); a row without any selected key (l = 0) gives 0
  const float inv_l = l > 0.f ? 1.f / l : 0.f;
  // O / l (and the gate) in the accumulator layout, written into the
  // staging tile at the gate values' places; then each row's 256 bytes go
  // out 4 rows per store instruction.  (With a single tile the gate loads
  // were issued in iteration 0 and may still be in flight.)
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  char* const xb = reinterpret_cast<char*>(dsm + kXBase + wu * 512);
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      uint2* const xp = reinterpret_cast<uint2*>(xb + xs_unit(i32, 4 * dt + r4) * 16 + 8 * h);
      float r[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) r[e] = round_bf16(o[dt][4 * r4 + e] * inv_l);
      if (p.flags & GSA_ATTN_OUT_GATE) {
        const uint2 gw = *xp;
        const float gl[4] = {bf16lo(gw.x), bf16hi(gw.x), bf16lo(gw.y), bf16hi(gw.y)};
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = round_bf16(r[e] * round_bf16(sigmoidf_fast(gl[e])));
      }
      *xp = uint2{pack_bf16(r[0], r[1]), pack_bf16(r[2], r[3])};
    }
  asm volatile("" ::: "memory");
  uint16_t* const ob = p.out + b * p.out_sb + hd * 128;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r = 4 * j + (lane >> 4), row = q0 + 32 * gw + r;
    const u32x4 v = xt[r * 16 + (lane & 15)];
    if (row < p.T)
      *reinterpret_cast<u32x4*>(ob + (int64_t)row * p.out_st + (((lane & 15) ^ (r & 15)) * 8)) = v;
  }
}

}  // namespace gsa

// ---------------------------------------------------------------------------
// Host entry points
// ---------------------------------------------------------------------------
using namespace gsa_host;

// Per device: the dense kernel's LDS limit has been raised.  (A benign race:
// concurrent first calls both set the same attribute.)
static constexpr int kMaxDevices = 64;
static bool g_dense_lds_set[kMaxDevices] = {};

namespace {
int prologue_vt_checks(const void* k, int64_t k_sb, int64_t k_st, const void* v, int64_t v_sb, int64_t v_st,
                       const void* vg, int64_t g_sb, int64_t g_st, const void* cos, const void* sin,
                       int64_t cs_st, int B, int T, int H, int d, int dtype, void* k_out, void* vt, int ldv) {
  if (!v || !vg || !vt) return GSA_ERR_NULL;
  if (k && (!cos || !sin || !k_out)) return GSA_ERR_NULL;
  if (dtype != GSA_DTYPE_BF16) return GSA_ERR_DTYPE;
  if (B < 1 || T < 1 || d != 128 || H < 1 || H > 64) return GSA_ERR_SHAPE;
  if (ldv < T || ldv % 64 != 0) return GSA_ERR_SHAPE;
  if ((int64_t)B * H * (ldv / 64) > 0x7fffffffLL) return GSA_ERR_SHAPE;
  if (!vec_ok(v, v_sb, v_st, dtype) || !vec_ok(vg, g_sb, g_st, dtype) || !aligned(vt, 16)) return GSA_ERR_ALIGN;
  if (k && (!vec_ok(k, k_sb, k_st, dtype) || !vec_ok(cos, 0, cs_st, dtype) || !vec_ok(sin, 0, cs_st, dtype) ||
            !aligned(k_out, 16)))
    return GSA_ERR_ALIGN;
  return GSA_OK;
}
}  // namespace

extern "C" int gsa_prologue_vt(const void* k, int64_t k_sb, int64_t k_st,
                               const void* v, int64_t v_sb, int64_t v_st,
                               const void* vg, int64_t g_sb, int64_t g_st,
                               const void* cos, const void* sin, int64_t cs_st,
                               int B, int T, int H, int d, int dtype,
                               void* k_out, void* vt, int ldv,
                               void* stream) {
  const int st = prologue_vt_checks(k, k_sb, k_st, v, v_sb, v_st, vg, g_sb, g_st, cos, sin, cs_st, B, T, H, d,
                                    dtype, k_out, vt, ldv);
  if (st) return st;
  gsa::ProVtArgs a{static_cast<const uint16_t*>(k), k_sb, k_st, static_cast<const uint16_t*>(v), v_sb, v_st,
                   static_cast<const uint16_t*>(vg), g_sb, g_st, static_cast<const uint16_t*>(cos),
                   static_cast<const uint16_t*>(sin), cs_st, static_cast<uint16_t*>(k_out),
                   static_cast<uint16_t*>(vt), T, H, ldv, ldv / 64};
  hipLaunchKernelGGL(gsa::prologue_vt_kernel, dim3(B * H * (ldv / 64)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
  return launch_status();
}

extern "C" int gsa_selection_mask(const int32_t* idx, int64_t i_sb, int64_t i_st, int k_sel,
                                  const int32_t* count, const uint8_t* mask,
                                  int B, int T, int Tkv, uint32_t* bits, int64_t b_sb, int64_t b_st,
                                  void* stream) {
  if (!idx || !bits) return GSA_ERR_NULL;
  if (B < 1 || T < 1 || Tkv < 1 || k_sel < 0) return GSA_ERR_SHAPE;
  const int W = 2 * ((Tkv + 63) / 64);
  if ((size_t)W * 4 > 65536) return GSA_ERR_SHAPE;
  if ((int64_t)B * T > 0x7fffffffLL) return GSA_ERR_SHAPE;
  if (!aligned(idx, 4) || !aligned(bits, 8) || (b_st % 2) || (b_sb % 2) || (count && !aligned(count, 4)))
    return GSA_ERR_ALIGN;
  hipLaunchKernelGGL(gsa::selection_mask_kernel, dim3(B * T), dim3(256), (size_t)W * 4,
                     static_cast<hipStream_t>(stream), idx, i_sb, i_st, k_sel, count, mask, T, Tkv, W, bits,
                     b_sb, b_st);
  return launch_status();
}

namespace {
// 32-row mask-operand groups of T query rows: whole 256-row blocks of the
// dense kernel (8 groups per block).
int64_t dense_groups(int T, int /*Tkv*/) {
  constexpr int w = gsa::kDenseWaves;
  return (int64_t)((T + 32 * w - 1) / (32 * w)) * w;
}
}  // namespace

// Mask operands: 1 KiB (64 lanes x 16 bytes) per (batch, 32-row group, 64-key
// tile); the groups are counted over whole query blocks of the dense kernel.
extern "C" size_t gsa_dense_attn_workspace_bytes(int B, int T, int Tkv) {
  if (B < 1 || T < 1 || Tkv < 1) return 0;
  return (size_t)B * (size_t)dense_groups(T, Tkv) * ((Tkv + 63) / 64) * 1024;
}

namespace {
// Checks shared by gsa_dense_lane_masks and gsa_dense_attn's mask step.
int lane_mask_checks(const uint32_t* bits, int64_t b_sb, int64_t b_st, int B, int T, int Tkv, const void* ws,
                     size_t ws_bytes) {
  if (!bits || !ws) return GSA_ERR_NULL;
  if (B < 1 || T < 1 || Tkv < 1) return GSA_ERR_SHAPE;
  const int NT = (Tkv + 63) / 64;
  if (b_st < 2 * NT || (B > 1 && b_sb < (int64_t)T * b_st)) return GSA_ERR_SHAPE;
  if (ws_bytes < gsa_dense_attn_workspace_bytes(B, T, Tkv)) return GSA_ERR_SHAPE;
  if ((int64_t)B * dense_groups(T, Tkv) * NT > 0x7fffffffLL) return GSA_ERR_SHAPE;
  // one thread per (row, kLmTiles tiles): the thread index stays 32-bit
  if ((int64_t)B * dense_groups(T, Tkv) * ((NT + gsa::kLmTiles - 1) / gsa::kLmTiles) * 32 > 0x7fffffffLL)
    return GSA_ERR_SHAPE;
  if (!aligned(bits, 8) || (b_sb % 2) || (b_st % 2) || !aligned(ws, 16)) return GSA_ERR_ALIGN;
  return GSA_OK;
}

gsa::LaneMaskArgs lane_mask_args(const uint32_t* bits, int64_t b_sb, int64_t b_st, int B, int T, int Tkv,
                                  int causal, void* ws) {
  const int NT = (Tkv + 63) / 64;
  const int G = (int)dense_groups(T, Tkv);
  const int nunits = B * G * ((NT + gsa::kLmTiles - 1) / gsa::kLmTiles);
  const int block_rows = causal ? 32 * gsa::kDenseWaves : 0;
  return gsa::LaneMaskArgs{bits, b_sb, b_st, T, G, NT, nunits, block_rows, static_cast<gsa::u32x4*>(ws)};
}

int launch_lane_masks(const uint32_t* bits, int64_t b_sb, int64_t b_st, int B, int T, int Tkv, int causal,
                      void* ws, hipStream_t s) {
  const gsa::LaneMaskArgs l = lane_mask_args(bits, b_sb, b_st, B, T, Tkv, causal, ws);
  hipLaunchKernelGGL(gsa::lane_mask_kernel, dim3((l.nunits + 7) / 8), dim3(256), 0, s, l);
  return launch_status();
}
}  // namespace

extern "C" int gsa_dense_lane_masks(const uint32_t* bits, int64_t b_sb, int64_t b_st, int B, int T, int Tkv,
                                    int causal, void* ws, size_t ws_bytes, void* stream) {
  const int st = lane_mask_checks(bits, b_sb, b_st, B, T, Tkv, ws, ws_bytes);
  if (st) return st;
  return launch_lane_masks(bits, b_sb, b_st, B, T, Tkv, causal, ws, static_cast<hipStream_t>(stream));
}

extern "C" int gsa_prologue_vt_lane_masks(const void* k, int64_t k_sb, int64_t k_st,
                                          const void* v, int64_t v_sb, int64_t v_st,
                                          const void* vg, int64_t g_sb, int64_t g_st,
                                          const void* cos, const void* sin, int64_t cs_st,
                                          int B, int T, int H, int d, int dtype,
                                          void* k_out, void* vt, int ldv,
                                          const uint32_t* bits, int64_t b_sb, int64_t b_st, int Tkv,
                                          int causal, void* ws, size_t ws_bytes, void* stream) {
  int st = prologue_vt_checks(k, k_sb, k_st, v, v_sb, v_st, vg, g_sb, g_st, cos, sin, cs_st, B, T, H, d, dtype,
                              k_out, vt, ldv);
  if (st) return st;
  if ((st = lane_mask_checks(bits, b_sb, b_st, B, T, Tkv, ws, ws_bytes))) return st;
  gsa::ProVtArgs a{static_cast<const uint16_t*>(k), k_sb, k_st, static_cast<const uint16_t*>(v), v_sb, v_st,
                   static_cast<const uint16_t*>(vg), g_sb, g_st, static_cast<const uint16_t*>(cos),
                   static_cast<const uint16_t*>(sin), cs_st, static_cast<uint16_t*>(k_out),
                   static_cast<uint16_t*>(vt), T, H, ldv, ldv / 64};
  const gsa::LaneMaskArgs l = lane_mask_args(bits, b_sb, b_st, B, T, Tkv, causal, ws);
  const int n_pro = B * H * (ldv / 64), n_lm = (l.nunits + 7) / 8;
  if ((int64_t)n_pro + n_lm > 0x7fffffffLL) return GSA_ERR_SHAPE;
  hipLaunchKernelGGL(gsa::prologue_vt_lane_mask_kernel, dim3(n_pro + n_lm), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a, l, n_pro, n_lm);
  return launch_status();
}

extern "C" int gsa_dense_attn(const void* q, int64_t q_sb, int64_t q_st,
                              const void* k, int64_t k_sb, int64_t k_st,
                              const void* vt, int64_t vt_sb, int64_t vt_sh, int ldv,
                              const uint32_t* bits, int64_t b_sb, int64_t b_st,
                              const void* og, int64_t o_sb, int64_t o_st,
                              const void* cos, const void* sin, int64_t cs_st,
                              void* out, int64_t out_sb, int64_t out_st,
                              int B, int T, int Tkv, int H, int d, float scale,
                              int dtype, int flags, int causal,
                              void* ws, size_t ws_bytes,
                              void* stream) {
  const bool ready = (flags & GSA_ATTN_MASKS_READY) != 0;
  if (!q || !k || !vt || !out || !ws || (!ready && !bits)) return GSA_ERR_NULL;
  if (flags & ~(GSA_ATTN_ROPE_Q | GSA_ATTN_OUT_GATE | GSA_ATTN_MASKS_READY | GSA_ATTN_ROPE_HALVES))
    return GSA_ERR_FLAGS;
  if ((flags & GSA_ATTN_ROPE_HALVES) && !(flags & GSA_ATTN_ROPE_Q)) return GSA_ERR_FLAGS;
  const bool halves = (flags & GSA_ATTN_ROPE_HALVES) != 0;
  if ((flags & GSA_ATTN_ROPE_Q) && (!cos || (!halves && !sin))) return GSA_ERR_NULL;
  if ((flags & GSA_ATTN_OUT_GATE) && !og) return GSA_ERR_NULL;
  if (dtype != GSA_DTYPE_BF16) return GSA_ERR_DTYPE;
  if (B < 1 || T < 1 || Tkv < 1 || d != 128 || H < 1 || H > 64) return GSA_ERR_SHAPE;
  const int NT = (Tkv + 63) / 64;
  if (ldv < NT * 64 || ldv % 64 != 0) return GSA_ERR_SHAPE;
  if (ws_bytes < gsa_dense_attn_workspace_bytes(B, T, Tkv)) return GSA_ERR_SHAPE;
  // per-lane load offsets within a tile are 32-bit byte offsets
  if (k_st > (1 << 24) || (int64_t)ldv > (1 << 23)) return GSA_ERR_SHAPE;
  // the staging tiles' row offsets (32 rows) are 32-bit byte offsets
  if (q_st > (1 << 24) || out_st > (1 << 24) || ((flags & GSA_ATTN_OUT_GATE) && o_st > (1 << 24)) ||
      ((flags & GSA_ATTN_ROPE_Q) && cs_st > (1 << 24)))
    return GSA_ERR_SHAPE;
  constexpr int W = gsa::kDenseWaves;         // waves per block: 32W query rows
  const int nqb = (T + 32 * W - 1) / (32 * W);
  const int64_t G = dense_groups(T, Tkv);      // 32-row groups, padded to whole blocks
  if ((int64_t)B * H * nqb > 0x7fffffffLL || B * G * NT > 0x7fffffffLL) return GSA_ERR_SHAPE;
  if (!vec_ok(q, q_sb, q_st, dtype) || !vec_ok(k, k_sb, k_st, dtype) || !vec_ok(vt, vt_sb, vt_sh, dtype) ||
      !vec_ok(out, out_sb, out_st, dtype) || !aligned(ws, 16))
    return GSA_ERR_ALIGN;
  if ((flags & GSA_ATTN_OUT_GATE) && !vec_ok(og, o_sb, o_st, dtype)) return GSA_ERR_ALIGN;
  if ((flags & GSA_ATTN_ROPE_Q) && (!vec_ok(cos, 0, cs_st, dtype) || (!halves && !vec_ok(sin, 0, cs_st, dtype))))
    return GSA_ERR_ALIGN;
  if (!ready) {
    const int st = lane_mask_checks(bits, b_sb, b_st, B, T, Tkv, ws, ws_bytes);
    if (st) return st;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const gsa::u32x4* lm = static_cast<const gsa::u32x4*>(ws);
  if (!ready) {
    const int st = launch_lane_masks(bits, b_sb, b_st, B, T, Tkv, causal, ws, s);
    if (st) return st;
  }
  flags &= ~GSA_ATTN_MASKS_READY;
  gsa::DenseArgs a{static_cast<const uint16_t*>(q), q_sb, q_st, static_cast<const uint16_t*>(k), k_sb, k_st,
                   static_cast<const uint16_t*>(vt), vt_sb, vt_sh, ldv, (int)G, NT,
                   static_cast<const uint16_t*>(og), o_sb, o_st, static_cast<const uint16_t*>(cos),
                   static_cast<const uint16_t*>(sin), cs_st, static_cast<uint16_t*>(out), out_sb, out_st,
                   B, T, Tkv, H, nqb, scale * gsa::kLog2e, flags | (causal ? gsa::kDenseCausal : 0)};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return GSA_ERR_SHAPE;
  if (!g_dense_lds_set[dev]) {   // more than the default 64 KiB of LDS per block
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(gsa::dense_attn_kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)gsa::kDenseLds);
    if (e != hipSuccess) return -static_cast<int>(e);
    g_dense_lds_set[dev] = true;
  }
  hipLaunchKernelGGL(gsa::dense_attn_kernel, dim3(B * H * nqb), dim3(64 * W), gsa::kDenseLds, s, a, lm);
  return launch_status();
}
