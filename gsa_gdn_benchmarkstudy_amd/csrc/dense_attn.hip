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
// Per block: one head, 256 query rows (8 waves of 32 rows; 384 rows in 12
// waves from 32K keys on), 64-key tiles in LDS.  With
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

// Waves per dense-attention block (32 query rows each): 8 for keys shorter
// than kDenseWideTkv, 12 from there on.  The lane-mask layout follows the
// same rule (its 32-row groups are padded to whole blocks), so producer and
// consumer agree from (T, Tkv) alone.
constexpr int kDenseWideTkv = 32768;
__host__ __device__ constexpr int dense_block_waves(int Tkv) { return Tkv >= kDenseWideTkv ? 12 : 8; }
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
// Selection bitmask -> per-lane masks of the dense kernel's score slots.
// For 32-row group g (rows 32g + i), 64-key tile kt and score slot
// s = 16c + r (c = 0,1; r = 0..15), lm[b][g][kt][s] bit (32h + i) is the
// selection bit of row 32g+i and key 64kt + 32c + 16(r/8) + 8h + r%8 -- the
// key that accumulator r of lane (h, i) holds in the S^T MFMA output of half
// c (see the key order below).  One wave per (b, g, 4 consecutive tiles):
// lane (h, i) reads row 32g+i's four 64-bit words and keeps keys 32h..32h+31
// of each; a 32x32 bit transpose in each half of the wave turns the rows into
// key columns (lane k: bit i = row 32g+i's bit of key k), and slot lane s
// takes its two columns; lanes 0..31 write each tile's 256 contiguous bytes.
// ---------------------------------------------------------------------------
constexpr int kLmTiles = 4;

// 32x32 bit transpose inside each 32-lane half of the wave: on entry lane i
// of a half holds row i (bit j = element (i, j)), on exit lane j holds
// column j (bit i = element (i, j)).  Stage b (16, 8, 4, 2, 1) swaps the
// off-diagonal b x b blocks of every 2b x 2b block between lanes i and i ^ b:
// the lane with bit b clear keeps the low b bits of each 2b-bit group and
// takes its partner's low ones, shifted up by b, into the high b; the other
// lane keeps the high b bits and takes its partner's high ones shifted down.
// Both shifts are one right rotation of the partner's word (by 32 - b or by
// b: the bits that wrap around land in the part the lane keeps), so a stage
// is a lane swizzle, a rotate and a bit select with per-lane constants.
struct BitTranspose {
  uint32_t keep[5], rot[5];   // per stage: bits the lane keeps, right rotation of the partner's word
  __device__ explicit BitTranspose(int lane) {
    constexpr uint32_t kLow[5] = {0x0000ffffu, 0x00ff00ffu, 0x0f0f0f0fu, 0x33333333u, 0x55555555u};
#pragma unroll
    for (int st = 0; st < 5; ++st) {
      const int b = 16 >> st;
      const bool up = (lane & b) != 0;
      keep[st] = up ? ~kLow[st] : kLow[st];
      rot[st] = up ? (uint32_t)b : (uint32_t)(32 - b);
    }
  }
  // ds_swizzle bit mode (and 0x1f, or 0, xor B): lane ^ B within its 32-lane half
  template <int St>
  __device__ __forceinline__ uint32_t stage(uint32_t x) const {
    constexpr int B = 16 >> St;
    const uint32_t y = (uint32_t)__builtin_amdgcn_ds_swizzle((int)x, (B << 10) | 0x1f);
    const uint32_t sh = __builtin_amdgcn_alignbit(y, y, rot[St]);
    return (x & keep[St]) | (sh & ~keep[St]);
  }
  __device__ __forceinline__ uint32_t operator()(uint32_t x) const {
    return stage<4>(stage<3>(stage<2>(stage<1>(stage<0>(x)))));
  }
};

struct LaneMaskArgs {
  const uint32_t* bits; int64_t b_sb, b_st;
  int T, G, NT, nwaves;
  int block_rows;   // causal: query rows per attention block (tiles past a block's last row are skipped); else 0
  uint64_t* lm;
};

// Block `blk` of the lane-mask pass: its 4 waves take waves 4*blk .. 4*blk+3.
__device__ __forceinline__ void lane_mask_block(const LaneMaskArgs& a, int blk) {
  const uint32_t* __restrict__ bits = a.bits;
  uint64_t* __restrict__ lm = a.lm;
  const int64_t b_sb = a.b_sb, b_st = a.b_st;
  const int T = a.T, G = a.G, NT = a.NT;
  const int wv = blk * 4 + (threadIdx.x >> 6);
  if (wv >= a.nwaves) return;
  const int nq = (NT + kLmTiles - 1) / kLmTiles;
  const int kq = wv % nq, bg = wv / nq;
  const int g = bg % G, b = bg / G;
  const int lane = threadIdx.x & 63, i = lane & 31, h = lane >> 5;
  const int row = 32 * g + i;
  const int kt0 = kq * kLmTiles;
  // Tiles the attention reads for this group: all of them, or (causal) those
  // up to the last row of the group's attention block, as its block does.
  int nt = NT;
  if (a.block_rows) nt = min(NT, ((32 * g) / a.block_rows + 1) * a.block_rows / kDK);
  if (kt0 >= nt) return;
  uint64_t words[kLmTiles];
  const uint64_t* src = reinterpret_cast<const uint64_t*>(bits + b * b_sb + (int64_t)min(row, T - 1) * b_st) + kt0;
#pragma unroll
  for (int u = 0; u < kLmTiles; ++u) words[u] = (row < T && kt0 + u < nt) ? src[u] : 0ull;
  // slot s = 16c + r (lane s < 32) holds key k0 = 32c + 16(r/8) + r%8 in its
  // low 32 bits (lanes h = 0) and key k0 + 8 in its high 32 bits (h = 1)
  const int s = lane & 31, k0 = 32 * (s >> 4) + 16 * ((s >> 3) & 1) + (s & 7);
  const BitTranspose transpose(lane);
#pragma unroll
  for (int u = 0; u < kLmTiles; ++u) {
    if (kt0 + u >= nt) break;
    uint64_t out = 0;
    // A tile no row of the group selects from (every tile past the group's
    // diagonal, for a causal selection) has all-zero masks: no transpose.
    if (ballot64(words[u] != 0ull)) {
      const uint32_t col = transpose((uint32_t)(words[u] >> (32 * h)));   // key `lane`'s column
      const uint32_t lo = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * k0, (int)col);
      const uint32_t hi = (uint32_t)__builtin_amdgcn_ds_bpermute(4 * (k0 + 8), (int)col);
      out = ((uint64_t)hi << 32) | lo;
    }
    if (lane < 32) lm[((int64_t)bg * NT + kt0 + u) * 32 + lane] = out;
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
// Block: W waves = 32W query rows of one head (wave w: rows 32w .. 32w+31):
// 8 waves (two per SIMD) or 12 (three per SIMD), by dense_block_waves.  K
// and V^T tiles reach LDS by direct global->LDS loads (16 B per lane; one
// instruction fills 1 KiB, lane-linear), K tiles and V^T tiles each through a
// pair of slots, in padded layouts (unit = 16 B = 8 bf16):
//   K   tile: 64 keys x 17 units, unit 16 of a key is padding
//   V^T tile: 128 rows x 9 units (64 keys), unit 8 of a row is padding
// The odd row strides make every MFMA operand read conflict-free (16 lanes
// reading one unit of 16 different rows hit 16 different bank groups), and
// each operand read is one base register plus an immediate offset.  Padding
// units receive a harmless duplicate load.
// Key order: in the S^T product of a 32-key half, MFMA row rho holds key
// pi(rho), pi swapping bits 2 and 3 of rho, so accumulator r of lane (h, i)
// holds key 16(r/8) + 8h + r%8.  A lane's 8 P values of each 16-key k-step
// are then contiguous keys, and its V^T operand is one 16-byte read.
//
// Tiles are pipelined (8 waves): S^T of tile t+1 is computed, one 32-key
// half at a time, while tile t's scores are masked half by half (each half
// with its own 16 lane-mask words), then the tile's one online-softmax
// decision with the lazy reference (below), then O^T += V^T(t) P^T(t) half by
// half, so MFMA and VALU work of one wave overlap.  12-wave blocks compute
// S^T(t) itself in that place (one S accumulator pair per wave).
// ---------------------------------------------------------------------------
struct DenseArgs {
  const uint16_t* q; int64_t q_sb, q_st;
  const uint16_t* k; int64_t k_sb, k_st;
  const uint16_t* vt; int64_t vt_sb, vt_sh; int ldv;
  int G, NT;                              // lane masks [B][G][NT][32] (kernel argument)
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
constexpr size_t kDenseLds = (size_t)2 * (kKU + kVU) * 16;   // two K slots, then two V^T slots

typedef float floatx16 __attribute__((ext_vector_type(16)));

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

// Pipeline of one block (W waves = 32W query rows of one head), tile t = 64
// keys.  K tiles and V^T tiles stream through separate pairs of LDS slots
// (tile t in slot t&1).  With PP (ping-pong S), iteration t, after one
// barrier:
//   loads  K(t+2) into K slot t&1 (S(t) was computed last iteration) and
//          V^T(t+1) into V slot (t+1)&1 (PV(t-1) is done);
//   MFMA   S^T(t+1) from K slot (t+1)&1, interleaved with the softmax of
//          S(t) (VALU), then O^T += V^T(t) P^T(t) from V slot t&1.
// So the S product of the next tile overlaps the softmax of this one, within
// the wave, at the cost of a second S accumulator pair (64 VGPRs).  Without
// PP, iteration t loads K(t+1) and V^T(t+1) into slots (t+1)&1 and computes
// S^T(t), its softmax and PV(t) from slots t&1: one S pair, so 12-wave blocks
// (three waves per SIMD) fit the register file, and the overlap of MFMA and
// VALU work comes from the other waves of the SIMD instead.  8 waves with PP
// is the faster form up to 16K keys, 12 without PP beyond (fewer tile loads
// per query row: at 65536 keys 17.1 -> 15.9 ms, K and V^T no longer fit the
// last-level cache).  Every load is issued one iteration before the barrier
// that publishes it; the loop is unrolled by two so that slot offsets are
// constants.
// lm is a separate restrict argument: nothing in this kernel writes it, and
// alias analysis can see that, so its uniform reads stay scalar loads.
template <int W, bool PP>
__global__ __launch_bounds__(64 * W, 1) void dense_attn_kernel(DenseArgs p, const uint64_t* __restrict__ lm) {
  extern __shared__ __align__(16) u32x4 dsm[];   // K slots 0, 1 (kKU units each), then V^T slots 0, 1 (kVU)
  constexpr int kDW = W;                          // waves per block
  constexpr int kDQ = 32 * W;                     // query rows per block
  constexpr int kDmaKW = (kDmaK + kDW - 1) / kDW;   // K instructions per wave (wave w: i = kDW*n + w < 17)
  constexpr int kDmaVW = (kDmaV + kDW - 1) / kDW;   // V^T instructions per wave

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int wu = __builtin_amdgcn_readfirstlane(w);
  const int i32 = lane & 31, h = lane >> 5;
  // heaviest query blocks first
  // Block order: batch by batch (the blocks in flight then share one
  // sequence's K and V^T, which stays in the last-level cache), within a
  // sequence the heaviest query blocks first, heads fastest.
  const int per_b = p.nqb * p.H;
  const int b = (int)(blockIdx.x / per_b);
  const int r2 = (int)(blockIdx.x % per_b);
  const int qb = p.nqb - 1 - r2 / p.H;
  const int hd = r2 % p.H;
  const int q0 = qb * kDQ;
  const int qrow = q0 + 32 * w + i32;
  const int qr = min(qrow, p.T - 1);

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
  // for the last tile, whose keys past Tkv-1 re-read key Tkv-1.
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
  // prologue loads: K(0), K(1) (ping-pong only), V(0)
  issue_k(kbase, 0, nkt == 1);
  if (PP && nkt > 1) issue_k(kbase + kstep, 1, nkt == 2);
  issue_v(vtb, 0);

  // ---- q: B operand of S^T; lane supplies d = 16s + 8h .. +7 of its row ----
  u32x4 qraw[8];
  const uint16_t* qp = p.q + b * p.q_sb + (int64_t)qr * p.q_st + hd * 128;
#pragma unroll
  for (int s = 0; s < 8; ++s) qraw[s] = *reinterpret_cast<const u32x4*>(qp + 16 * s + 8 * h);
  if (p.flags & GSA_ATTN_ROPE_Q) {
    // rotate_half partner of d (d < 64: -x[d+64]; else x[d-64]) is register s^4
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      float c0[8], s0[8], c1[8], s1[8];
      load8(p.cos + (int64_t)qr * p.cs_st + 16 * s + 8 * h, c0);
      load8(p.sin + (int64_t)qr * p.cs_st + 16 * s + 8 * h, s0);
      load8(p.cos + (int64_t)qr * p.cs_st + 16 * (s + 4) + 8 * h, c1);
      load8(p.sin + (int64_t)qr * p.cs_st + 16 * (s + 4) + 8 * h, s1);
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

  floatx16 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dt][r] = 0.f;
  // softmax state of the lane's row: reference m (log2 domain), m + kLazy,
  // -m (0 while m = -inf), and the running sum l
  float m = -__builtin_inff(), mlz = -__builtin_inff(), nm = 0.f, l = 0.f;
  const bf16x2 ones2 = __builtin_bit_cast(bf16x2, 0x3f803f80u);   // (1, 1)

  // this wave's lane masks: group kDW*qb + w (wave index uniform for scalar loads)
  const uint64_t* lmw = lm + ((int64_t)b * p.G + kDW * qb + wu) * p.NT * 32;
  // operand read offsets (units within a slot): K row of MFMA row i32, V^T row i32
  const int kread = swap_bits23(i32) * kKRow + h;
  const int vread = 2 * kKU + i32 * kVRow + h;

  // S^T of one 32-key half of the tile in K slot ks
  auto s_half = [&](int ks, int c) {
    const u32x4* sK = dsm + ks * kKU + kread;
    bf16x8 f[8];
#pragma unroll
    for (int s = 0; s < 8; ++s) f[s] = __builtin_bit_cast(bf16x8, sK[32 * c * kKRow + 2 * s]);
    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
    for (int s = 0; s < 8; ++s) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[s], qop[s], acc, 0, 0, 0);
    return acc;
  };
  // Masked online softmax, one step per 64-key tile: p = 2^(s*scale*log2e -
  // m) against a per-row reference m that only moves when the tile's row max
  // exceeds it by more than kLazy (p <= 2^kLazy; out = O / l does not depend
  // on m).  mask_half keeps the selected scores of one 32-key half (the others
  // -inf) and returns their max; both halves are masked before the tile's one
  // reference decision, so their lane-mask loads and the S^T MFMAs of the next
  // tile share one stretch of code.  A move is rare: its bookkeeping --
  // alpha = 2^(m_old - m_new), O and l times alpha, the new m, m + kLazy and
  // -m -- runs in a branch the wave takes only when one of its rows moves.
  // exp_half turns a half's scores into P (two B operands of O^T) and adds
  // the bf16 values that the PV product uses to l, one dot2 per pair.
  // (mask_half_r takes the half's 16 mask words from registers, mask_half
  // loads them from the lane-mask array where they are used)
  auto mask_half_r = [&](const floatx16& acc, const uint64_t (&mw)[16], float (&sv)[16]) -> float {
    float mx = -__builtin_inff();
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const bool sel = __builtin_amdgcn_inverse_ballot_w64(mw[r]);
      sv[r] = sel ? acc[r] : -__builtin_inff();
      mx = fmaxf(mx, sv[r]);
    }
    return mx;                                      // never NaN: the max is seeded with -inf
  };
  auto mask_half = [&](const floatx16& acc, const uint64_t* lmt, int c, float (&sv)[16]) -> float {
    float mx = -__builtin_inff();
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const bool sel = __builtin_amdgcn_inverse_ballot_w64(lmt[16 * c + r]);
      sv[r] = sel ? acc[r] : -__builtin_inff();
      mx = fmaxf(mx, sv[r]);
    }
    return mx;                                      // never NaN: the max is seeded with -inf
  };
  auto exp_half = [&](const float (&sv)[16], uint32_t (&pk)[2][4]) {
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      const float p0 = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[r], p.scale_l2, nm));
      const float p1 = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[r + 1], p.scale_l2, nm));
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
  const char* vsrc = vtb + kDK * 2;                  // V^T tile kt+1
  const uint64_t* lmt = lmw;                         // lane masks of tile kt
  // The first half's 16 lane-mask words of a tile are loaded one iteration
  // ahead, after the previous tile's masks are used, so their scalar loads
  // are in flight during the PV products and done at the next barrier (at
  // T=65536 the masks come from HBM; with 8-wave blocks 18.3 -> 17.0 ms).
  // The second half's are loaded where they are used: holding both halves
  // ahead would need 32 more SGPRs and spills 130 of them.
  uint64_t mw0[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) mw0[r] = lmw[r];
  // Tile kt once both halves are masked (scores sv0, sv1, maxima mx0, mx1):
  // the softmax decision, P, O^T += V^T(kt) P^T(kt) from V slot vs, and the
  // next tile's first-half mask words.
  auto softmax_pv = [&](int kt, int vs, float mx0, float mx1, const float (&sv0)[16], const float (&sv1)[16]) {
    const float mx = max_halves(mx1 > mx0 ? mx1 : mx0) * p.scale_l2;
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
    exp_half(sv0, pk0);
    pv_half(vs, 0, pk0);
    exp_half(sv1, pk1);
    pv_half(vs, 1, pk1);
    if (kt + 1 < nkt) {
#pragma unroll
      for (int r = 0; r < 16; ++r) mw0[r] = lmt[32 + r];
    }
    lmt += 32;
  };

  if constexpr (PP) {
    // S^T of tile kt in sc[kt & 1]: with the loop unrolled by two, each
    // iteration writes the other pair, so no accumulator is copied
    floatx16 sc[2][2];
    sc[0][0] = s_half(0, 0);
    sc[0][1] = s_half(0, 1);                        // S^T of tile 0
    const char* ksrc = kbase + 2 * kstep;            // K tile kt+2
    // one iteration; P = kt & 1
    auto step = [&](int kt, auto par) {
      constexpr int P = decltype(par)::value;
      // this wave's loads of K(kt+1) and V^T(kt) (issued last iteration) are
      // done and its LDS reads have returned; the barrier publishes every
      // wave's loads and frees K slot P and V slot 1-P
      asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      if (kt + 2 < nkt) issue_k(ksrc, P, kt + 3 == nkt);
      if (kt + 1 < nkt) issue_v(vsrc, 1 - P);
      ksrc += kstep;
      vsrc += kDK * 2;

      float sv0[16], sv1[16];
      sc[1 - P][0] = s_half(1 - P, 0);             // S^T(kt+1) || softmax(kt); stale on the last tile, unused
      const float mx0 = mask_half_r(sc[P][0], mw0, sv0);
      sc[1 - P][1] = s_half(1 - P, 1);
      const float mx1 = mask_half(sc[P][1], lmt, 1, sv1);
      softmax_pv(kt, P, mx0, mx1, sv0, sv1);
    };
    int t = 0;
    for (; t + 1 < nkt; t += 2) {
      step(t, Int<0>{});
      step(t + 1, Int<1>{});
    }
    if (t < nkt) step(t, Int<0>{});
  } else {
    const char* ksrc = kbase + kstep;                // K tile kt+1
    // one iteration; P = kt & 1
    auto step = [&](int kt, auto par) {
      constexpr int P = decltype(par)::value;
      // this wave's loads of K(kt) and V^T(kt) (issued last iteration) are
      // done and its LDS reads have returned; the barrier publishes every
      // wave's loads and frees slots 1-P (tile kt-1) for tile kt+1
      asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      if (kt + 1 < nkt) {
        issue_k(ksrc, 1 - P, kt + 2 == nkt);
        issue_v(vsrc, 1 - P);
      }
      ksrc += kstep;
      vsrc += kDK * 2;

      float sv0[16], sv1[16];
      const floatx16 s0 = s_half(P, 0);
      const float mx0 = mask_half_r(s0, mw0, sv0);
      const floatx16 s1 = s_half(P, 1);
      const float mx1 = mask_half(s1, lmt, 1, sv1);
      softmax_pv(kt, P, mx0, mx1, sv0, sv1);
    };
    int t = 0;
    for (; t + 1 < nkt; t += 2) {
      step(t, Int<0>{});
      step(t + 1, Int<1>{});
    }
    if (t < nkt) step(t, Int<0>{});
  }

  // ---- epilogue: normalise, bf16, optional output gate ----
  l = sum_halves(l);
  // O / l as O * (1/l): one division per row instead of one per element
  // (the product is within 1.5 fp32 ulp of the quotient before the bf16
  // rounding); a row without any selected key (l = 0) gives 0
  const float inv_l = l > 0.f ? 1.f / l : 0.f;
  if (qrow < p.T) {
    uint16_t* op = p.out + b * p.out_sb + (int64_t)qrow * p.out_st + hd * 128;
    const uint16_t* gp = (p.flags & GSA_ATTN_OUT_GATE) ? p.og + b * p.o_sb + (int64_t)qrow * p.o_st + hd * 128
                                                       : nullptr;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int d0 = 32 * dt + 8 * r4 + 4 * h;
        float r[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) r[e] = round_bf16(o[dt][4 * r4 + e] * inv_l);
        if (gp) {
          const uint2 gw = *reinterpret_cast<const uint2*>(gp + d0);
          const float gl[4] = {bf16lo(gw.x), bf16hi(gw.x), bf16lo(gw.y), bf16hi(gw.y)};
#pragma unroll
          for (int e = 0; e < 4; ++e) r[e] = round_bf16(r[e] * round_bf16(sigmoidf_fast(gl[e])));
        }
        *reinterpret_cast<uint2*>(op + d0) = uint2{pack_bf16(r[0], r[1]), pack_bf16(r[2], r[3])};
      }
  }
}

}  // namespace gsa

// ---------------------------------------------------------------------------
// Host entry points
// ---------------------------------------------------------------------------
using namespace gsa_host;

// Per device and dense kernel (8 waves, 12 waves): its LDS limit has been
// raised.  (A benign race: concurrent first calls both set the same
// attribute.)
static constexpr int kMaxDevices = 64;
static bool g_dense_lds_set[kMaxDevices][2] = {};

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
// 32-row lane-mask groups of T query rows: whole blocks of the dense kernel
// that runs for Tkv keys (8 groups per block, 12 from 32K keys on).
int64_t dense_groups(int T, int Tkv) {
  const int w = gsa::dense_block_waves(Tkv);
  return (int64_t)((T + 32 * w - 1) / (32 * w)) * w;
}
}  // namespace

// Lane masks: 32 per (batch, 32-row group, 64-key tile); the groups are
// counted over whole query blocks of the dense kernel.
extern "C" size_t gsa_dense_attn_workspace_bytes(int B, int T, int Tkv) {
  if (B < 1 || T < 1 || Tkv < 1) return 0;
  return (size_t)B * (size_t)dense_groups(T, Tkv) * ((Tkv + 63) / 64) * 32 * sizeof(uint64_t);
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
  if (!aligned(bits, 8) || (b_sb % 2) || (b_st % 2) || !aligned(ws, 8)) return GSA_ERR_ALIGN;
  return GSA_OK;
}

gsa::LaneMaskArgs lane_mask_args(const uint32_t* bits, int64_t b_sb, int64_t b_st, int B, int T, int Tkv,
                                  int causal, void* ws) {
  const int NT = (Tkv + 63) / 64;
  const int G = (int)dense_groups(T, Tkv);
  const int nwaves = B * G * ((NT + gsa::kLmTiles - 1) / gsa::kLmTiles);
  const int block_rows = causal ? 32 * gsa::dense_block_waves(Tkv) : 0;
  return gsa::LaneMaskArgs{bits, b_sb, b_st, T, G, NT, nwaves, block_rows, static_cast<uint64_t*>(ws)};
}

int launch_lane_masks(const uint32_t* bits, int64_t b_sb, int64_t b_st, int B, int T, int Tkv, int causal,
                      void* ws, hipStream_t s) {
  const gsa::LaneMaskArgs l = lane_mask_args(bits, b_sb, b_st, B, T, Tkv, causal, ws);
  hipLaunchKernelGGL(gsa::lane_mask_kernel, dim3((l.nwaves + 3) / 4), dim3(256), 0, s, l);
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
  const int n_pro = B * H * (ldv / 64), n_lm = (l.nwaves + 3) / 4;
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
  if (flags & ~(GSA_ATTN_ROPE_Q | GSA_ATTN_OUT_GATE | GSA_ATTN_MASKS_READY)) return GSA_ERR_FLAGS;
  if ((flags & GSA_ATTN_ROPE_Q) && (!cos || !sin)) return GSA_ERR_NULL;
  if ((flags & GSA_ATTN_OUT_GATE) && !og) return GSA_ERR_NULL;
  if (dtype != GSA_DTYPE_BF16) return GSA_ERR_DTYPE;
  if (B < 1 || T < 1 || Tkv < 1 || d != 128 || H < 1 || H > 64) return GSA_ERR_SHAPE;
  const int NT = (Tkv + 63) / 64;
  if (ldv < NT * 64 || ldv % 64 != 0) return GSA_ERR_SHAPE;
  if (ws_bytes < gsa_dense_attn_workspace_bytes(B, T, Tkv)) return GSA_ERR_SHAPE;
  // per-lane load offsets within a tile are 32-bit byte offsets
  if (k_st > (1 << 24) || (int64_t)ldv > (1 << 23)) return GSA_ERR_SHAPE;
  const int W = gsa::dense_block_waves(Tkv);   // waves per block: 32W query rows
  const int nqb = (T + 32 * W - 1) / (32 * W);
  const int64_t G = dense_groups(T, Tkv);      // 32-row groups, padded to whole blocks
  if ((int64_t)B * H * nqb > 0x7fffffffLL || B * G * NT > 0x7fffffffLL) return GSA_ERR_SHAPE;
  if (!vec_ok(q, q_sb, q_st, dtype) || !vec_ok(k, k_sb, k_st, dtype) || !vec_ok(vt, vt_sb, vt_sh, dtype) ||
      !vec_ok(out, out_sb, out_st, dtype) || !aligned(ws, 8))
    return GSA_ERR_ALIGN;
  if ((flags & GSA_ATTN_OUT_GATE) && !vec_ok(og, o_sb, o_st, dtype)) return GSA_ERR_ALIGN;
  if ((flags & GSA_ATTN_ROPE_Q) && (!vec_ok(cos, 0, cs_st, dtype) || !vec_ok(sin, 0, cs_st, dtype)))
    return GSA_ERR_ALIGN;
  if (!ready) {
    const int st = lane_mask_checks(bits, b_sb, b_st, B, T, Tkv, ws, ws_bytes);
    if (st) return st;
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint64_t* lm = static_cast<uint64_t*>(ws);
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
  const bool wide = W == 12;
  const void* fn = wide ? reinterpret_cast<const void*>(gsa::dense_attn_kernel<12, false>)
                        : reinterpret_cast<const void*>(gsa::dense_attn_kernel<8, true>);
  if (!g_dense_lds_set[dev][wide]) {   // more than the default 64 KiB of LDS per block
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)gsa::kDenseLds);
    if (e != hipSuccess) return -static_cast<int>(e);
    g_dense_lds_set[dev][wide] = true;
  }
  if (wide)
    hipLaunchKernelGGL((gsa::dense_attn_kernel<12, false>), dim3(B * H * nqb), dim3(64 * 12), gsa::kDenseLds, s,
                       a, static_cast<const uint64_t*>(lm));
  else
    hipLaunchKernelGGL((gsa::dense_attn_kernel<8, true>), dim3(B * H * nqb), dim3(64 * 8), gsa::kDenseLds, s, a,
                       static_cast<const uint64_t*>(lm));
  return launch_status();
}
