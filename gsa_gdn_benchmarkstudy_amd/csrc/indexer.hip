// Gated lightning indexer on gfx950 MFMA, and its fused exact top-k select.
//
//   S[b,i,j] = sum_h sigmoid(w[b,i,h]) * sigmoid(scale*<q[b,i,h,:], k[b,j,:]> + bias[h])
//
// (semantics of gsa_triton/gsa_ref.py:97-126).  Both kernels below share one
// score routine -- the same MFMA sequence and the same epilogue instructions
// -- so a score is bit-identical wherever it is computed; the fused selector
// relies on that to recompute scores pass after pass.
//
// Tiling: one wave owns 16 query rows.  Its MFMA A operand (q, 4 heads x 64
// dims) stays in registers for the whole kernel; keys stream through in tiles
// of 16, each tile one 16x16 output block per head:
//   bf16: v_mfma_f32_16x16x32_bf16, 2 k-steps per head  (8 MFMA per tile)
//   fp32: v_mfma_f32_16x16x4_f32,  16 k-steps per head (64 MFMA per tile)
// Output layout of a 16x16 block: lane l holds rows 4*(l/16)+e (e = 0..3) of
// column l%16.
#include "gsa_common.h"

#pragma clang fp contract(off)

namespace gsa {

constexpr int kHi = 4;    // indexer heads
constexpr int kDi = 64;   // indexer head dim

template <typename T> struct Mfma;

template <> struct Mfma<uint16_t> {
  static constexpr int kSteps = 2;          // 64 dims / 32 per MFMA
  typedef bf16x8 Op;
  // lane group g = lane/16 supplies k = 32*s + 8*g .. +7 of its row/column
  __device__ static Op load(const uint16_t* rowp, int off, int s, int g) {
    return *reinterpret_cast<const bf16x8*>(rowp + off + s * 32 + g * 8);
  }
  __device__ static floatx4 mma(Op a, Op b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <> struct Mfma<float> {
  static constexpr int kSteps = 16;         // 64 dims / 4 per MFMA
  typedef float Op;
  __device__ static Op load(const float* rowp, int off, int s, int g) {
    return rowp[off + s * 4 + g];
  }
  __device__ static floatx4 mma(Op a, Op b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

struct IdxArgs {
  const void* q; int64_t q_sb, q_st;
  const void* k; int64_t k_sb, k_st;
  const void* w; int64_t w_sb, w_st;
  const float* bias;    // device fp32 [Hi]
  float scale_l2;       // -scale * log2(e)
  int B, T;
};

// Per-lane state of one wave's 16-row group.
template <typename T>
struct RowGroup {
  typename Mfma<T>::Op qa[kHi][Mfma<T>::kSteps];  // A operand: row r0 + lane%16
  float a[4][kHi];                                // sigmoid(w) of rows r0 + 4*(lane/16) + e
  float bias_l2[kHi];                             // -bias[h] * log2(e)
  float scale_l2;                                 // -scale * log2(e)
  const T* kbase;                                 // k_idx of this batch
  int64_t k_st;

  __device__ void init(const IdxArgs& p, int b, int r0, int lane) {
    const int g = lane >> 4, lr = lane & 15;
    const T* qb = static_cast<const T*>(p.q) + b * p.q_sb;
    const int qrow = min(r0 + lr, p.T - 1);
    const T* qrp = qb + (int64_t)qrow * p.q_st;
#pragma unroll
    for (int h = 0; h < kHi; ++h)
#pragma unroll
      for (int s = 0; s < Mfma<T>::kSteps; ++s) qa[h][s] = Mfma<T>::load(qrp, h * kDi, s, g);
    const T* wb = static_cast<const T*>(p.w) + b * p.w_sb;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = min(r0 + 4 * g + e, p.T - 1);
#pragma unroll
      for (int h = 0; h < kHi; ++h) {
        const T wv = wb[(int64_t)row * p.w_st + h];
        float wf;
        if constexpr (Elem<T>::kBf16) wf = __uint_as_float((uint32_t)wv << 16);
        else wf = wv;
        a[e][h] = sigmoidf_fast(wf);
      }
    }
    kbase = static_cast<const T*>(p.k) + b * p.k_sb;
    k_st = p.k_st;
#pragma unroll
    for (int h = 0; h < kHi; ++h) bias_l2[h] = -p.bias[h] * kLog2e;
    scale_l2 = p.scale_l2;
  }

  // B operand of key tile [j0, j0+16): column lane%16, clamped to a valid row.
  __device__ void load_keys(int j0, int T_, int lane, typename Mfma<T>::Op (&kb)[Mfma<T>::kSteps]) const {
    const int j = min(j0 + (lane & 15), T_ - 1);
    const T* krp = kbase + (int64_t)j * k_st;
#pragma unroll
    for (int s = 0; s < Mfma<T>::kSteps; ++s) kb[s] = Mfma<T>::load(krp, 0, s, lane >> 4);
  }

  __device__ void mma(const typename Mfma<T>::Op (&kb)[Mfma<T>::kSteps], floatx4 (&acc)[kHi]) const {
#pragma unroll
    for (int h = 0; h < kHi; ++h) {
      floatx4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < Mfma<T>::kSteps; ++s) c = Mfma<T>::mma(qa[h][s], kb[s], c);
      acc[h] = c;
    }
  }

  // Fused epilogue for output slot e: sum_h a_h * sigmoid(scale*dot_h + bias_h).
  __device__ float score(const floatx4 (&acc)[kHi], int e) const {
    float s = 0.f;
#pragma unroll
    for (int h = 0; h < kHi; ++h) {
      const float t = __builtin_fmaf(acc[h][e], scale_l2, bias_l2[h]);
      const float r = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t));
      s = (h == 0) ? a[e][h] * r : __builtin_fmaf(a[e][h], r, s);
    }
    return s;
  }
};

// ---------------------------------------------------------------------------
// Full score matrix (the fused_gated_indexer API).  4 waves per block, one
// 16-row group per wave; causal tiles above the diagonal are filled with -inf
// without computing them.
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void indexer_scores_kernel(IdxArgs p, int causal, float* S,
                                                             int64_t s_sb, int64_t s_st) {
  const int lane = threadIdx.x & 63;
  const int ngroups = (p.T + 15) >> 4;
  const int wv = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wv >= p.B * ngroups) return;
  const int b = wv / ngroups;
  const int r0 = (wv % ngroups) * 16;
  const int g = lane >> 4, lr = lane & 15;

  RowGroup<T> rg;
  rg.init(p, b, r0, lane);
  float* Sb = S + b * s_sb;

  const int jend = causal ? min(p.T, r0 + 16) : p.T;
  typename Mfma<T>::Op kb[Mfma<T>::kSteps], kn[Mfma<T>::kSteps];
  rg.load_keys(0, p.T, lane, kn);
  for (int j0 = 0; j0 < jend; j0 += 16) {
#pragma unroll
    for (int s = 0; s < Mfma<T>::kSteps; ++s) kb[s] = kn[s];
    if (j0 + 16 < jend) rg.load_keys(j0 + 16, p.T, lane, kn);
    floatx4 acc[kHi];
    rg.mma(kb, acc);
    const int col = j0 + lr;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = r0 + 4 * g + e;
      if (row < p.T && col < p.T) {
        const float sc = (causal && col > row) ? -__builtin_inff() : rg.score(acc, e);
        Sb[(int64_t)row * s_st + col] = sc;
      }
    }
  }
  for (int j0 = ((jend + 15) >> 4) << 4; j0 < p.T; j0 += 16) {
    const int col = j0 + lr;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int row = r0 + 4 * g + e;
      if (row < p.T && col < p.T) Sb[(int64_t)row * s_st + col] = -__builtin_inff();
    }
  }
}

// ---------------------------------------------------------------------------
// Fused indexer + exact top-k.
//
// Output: the selection as a bitmask, bits[b][t] bit j set iff key j is one
// of row t's selected keys (W = 2*ceil(T/64) uint32 words per row; words past
// row t's causal range are zero).  One 512-thread block per 16-row group,
// heaviest groups first; its 8 waves take the group's causal 16-key tiles
// round-robin and share the row state in LDS (8 rather than 4 waves halve
// the time of the heaviest groups, which bound the kernel when the whole
// grid fits the GPU at once).  Rows with t+1 <= k select
// every causal key.  For the others:
//   pass 1  MFMA scores -> value-linear histogram, bin = floor(s * NB /
//           sum_h sigmoid(w_h)), and every score tile is stored to the
//           workspace -> the bin b1 holding the k-th largest score and the
//           rank of the k-th largest inside it;
//   pass 2  the stored scores are read back: entries in bins above b1 are
//           selected (ballots -> one 64-bit word of the row's bitmask per 4
//           tiles); entries in b1 (at most kWCap per row and wave) are
//           collected as (key, index);
//   resolve exact MSB-first radix select among a row's candidates -> the
//           threshold key theta and how many entries equal to theta to take,
//           lowest indices first; winning candidates are OR-ed into the mask.
// A bin holding more candidates than fit (degenerate scores, e.g. all equal)
// falls back to four 8-bit radix passes over the stored scores of the bin,
// then one ordered pass by a single wave marks the winners.
//
// Workspace: group g of batch b owns (g+1) consecutive 1 KiB score tiles
// starting at tile b*tri(G) + tri(g), tri(n) = n(n+1)/2, G = ceil(T/16);
// lane l of the wave that computes a tile stores its four output slots
// (rows 4*(l/16)+e, column l%16) as floats 4l .. 4l+3, the layout it reads
// back.  After the score tiles, block i owns 16 x kCap (key, index) slots
// for its rows' candidates (kept out of LDS, so that a block needs only its
// 17 KiB of histograms and can share a CU with a GEMM block).
// ---------------------------------------------------------------------------
constexpr int kNB = 512;                 // histogram bins per row
constexpr int kGroupWaves = 8;           // waves per 16-row group
constexpr int kGroupThreads = 64 * kGroupWaves;
constexpr int kWCap = 128;               // candidates per row and wave
constexpr int kCap = kWCap * kGroupWaves;  // candidates per row

// Per-row histogram in LDS.  Packed: 512 bins as 16-bit counts, two per
// word (exact while a row has at most 65535 keys, i.e. T <= 65535), 17 KiB
// for the block -- small enough for a block to share a CU with the
// projection GEMM's.  Unpacked: 32-bit counts.  Bin kNB is a trash bin
// (invalid slots) in the row's padding word, which no scan reads; the odd
// row strides put one bin of the 16 rows in distinct banks.  The overflow
// path's 256-bin digit histograms use 32-bit words with either stride.
template <bool kPacked>
struct Hist {
  static constexpr int kStride = kPacked ? kNB / 2 + 1 : kNB + 1;
  __device__ static void add(uint32_t* row, int bin) {
    if constexpr (kPacked) atomicAdd(&row[bin >> 1], 1u << (16 * (bin & 1)));
    else atomicAdd(&row[bin], 1u);
  }
  __device__ static int count(const uint32_t* row, int bin) {
    if constexpr (kPacked) return (int)((row[bin >> 1] >> (16 * (bin & 1))) & 0xffffu);
    else return (int)row[bin];
  }
};
constexpr int kTile = 256;               // floats per stored 16x16 score tile

enum RowMode : int { kNone = 0, kTrivial = 1, kActive = 2, kResolved = 3, kOverflow = 4 };

__device__ __forceinline__ int bin_of(float s, float inv_w) {
  return (int)fmaxf(0.f, fminf(s * inv_w, (float)(kNB - 1)));
}

// Causal-prefix chunk of row `row` for 16-key tile `tile`: keys <= row set.
__device__ __forceinline__ uint16_t prefix_chunk(int row, int tile) {
  const int n = row - 16 * tile + 1;    // keys of this tile at or before the row
  return n >= 16 ? (uint16_t)0xffffu : (n <= 0 ? (uint16_t)0 : (uint16_t)((1u << n) - 1u));
}

// Selection parameters of one launch.  The kernel runs in one of three phases:
//   0  fused: every row takes k = k_eff (the reference selector);
//   1  variance-adaptive k, first launch: pass 1 only, then each row's
//      population variance of its causal scores -> row_var, and the block's
//      histograms -> hist (scores stay in the workspace);
//   2  variance-adaptive k, second launch: row t takes k = k_rows[b*T+t]; the
//      histograms come back from hist instead of pass 1, then pass 2,
//      resolve and overflow as in phase 0.
// k_rows is written between the two launches by adaptive_k_kernel, which
// needs every row's variance (its mean over all rows is global).
struct SelArgs {
  int k_eff;              // phase 0
  const int* k_rows;      // phase 2: [B*T]
  float* row_var;         // phase 1: [B*T]
  uint32_t* hist;         // phases 1, 2: 16 * Hist::kStride words per block
};

template <typename T, bool kPacked, int kPhase>
__global__ __launch_bounds__(kGroupThreads) void indexer_bits_kernel(IdxArgs p, SelArgs sa, uint32_t* bits,
                                                           int64_t b_sb, int64_t b_st, float* ws, uint2* ws_cand) {
  using H = Hist<kPacked>;
  constexpr int kHStride = H::kStride;
  __shared__ uint32_t sh[16 * kHStride];   // histograms
  __shared__ uint32_t sh_wcnt[16 * kGroupWaves];
  __shared__ int st_mode[16], st_b1[16], st_need[16];
  __shared__ uint32_t st_key[16];
  __shared__ int st_any[2];                // [0] any active row, [1] any overflow

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, lr = lane & 15;
  const int ngroups = (p.T + 15) >> 4;
  const int b = blockIdx.x % p.B;
  const int rg_idx = ngroups - 1 - blockIdx.x / p.B;
  const int r0 = rg_idx * 16;
  uint32_t* bbase = bits + b * b_sb;
  uint16_t* b16 = reinterpret_cast<uint16_t*>(bbase);
  const int64_t row16 = 2 * b_st;          // uint16 chunks per row
  float* wsg = ws + ((int64_t)b * ngroups * (ngroups + 1) / 2 + (int64_t)rg_idx * (rg_idx + 1) / 2) * kTile;
  // this block's candidates (key, index): row rl, wave w, slot i at [rl][w * kWCap + i]
  uint2* cand = ws_cand + (int64_t)blockIdx.x * 16 * kCap;

  if (tid < 16) {
    const int row = r0 + tid;
    int k = sa.k_eff;
    if constexpr (kPhase == 2) k = row < p.T ? sa.k_rows[(int64_t)b * p.T + row] : 1;
    // phase 1 scores every row (each row's variance enters the global mean)
    st_mode[tid] = row >= p.T ? kNone : ((kPhase == 1 || row + 1 > k) ? kActive : kTrivial);
    st_need[tid] = k;
  }
  if (tid < 2) st_any[tid] = 0;
  __syncthreads();
  if (tid < 16 && st_mode[tid] == kActive) st_any[0] = 1;

  // Every chunk after the diagonal tile is zero; trivial rows get their
  // causal prefix now.  (The zeroing is largest for the lightest groups.)
  // Phase 1 writes no mask.
  const int ntl = rg_idx + 1;                  // causal 16-key tiles 0 .. rg_idx
  const int zend = (rg_idx | 3) + 1;           // chunks up to the end of the 64-key tile
  if (kPhase != 1) {
    for (int i = tid; i < 16 * zend; i += kGroupThreads) {
      const int rl = i / zend, tile = i % zend;
      const int row = r0 + rl;
      if (row >= p.T) continue;
      if (tile >= ntl) b16[row * row16 + tile] = 0;
      else if (st_mode[rl] == kTrivial) b16[row * row16 + tile] = prefix_chunk(row, tile);
    }
    const int W = 2 * ((p.T + 63) >> 6);
    const int d0 = zend >> 2;                    // first 8-byte pair of words past the 64-key tile
    const int npair = (W >> 1) - d0;
    for (int i = tid; i < 16 * npair; i += kGroupThreads) {
      const int rl = i / npair, pr = d0 + i % npair;
      const int row = r0 + rl;
      if (row < p.T) reinterpret_cast<uint2*>(bbase + (int64_t)row * b_st)[pr] = uint2{0u, 0u};
    }
  }
  __syncthreads();
  if (!st_any[0]) return;

  RowGroup<T> rgp;
  rgp.init(p, b, r0, lane);
  bool act[4];
  int b1[4];
  float inv_w[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    act[e] = st_mode[4 * g + e] == kActive;
    const float smax = ((rgp.a[e][0] + rgp.a[e][1]) + rgp.a[e][2]) + rgp.a[e][3];
    inv_w[e] = (float)kNB / (smax * 1.0009765625f + 1e-30f);
    b1[e] = 0;
  }
  // Lane 16g+e (e < 4) writes the mask chunks of row 4g+e.
  const int own_row = r0 + 4 * g + (lr & 3);
  const bool own_act = lr < 4 && st_mode[4 * g + (lr & 3)] == kActive;
  auto slot_valid = [&](int col, bool (&valid)[4]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) valid[e] = act[e] && col <= r0 + 4 * g + e;
  };

  // ---- pass 1: scores -> histogram + workspace ------------------------------
  // This wave's tiles: wave, wave+4, ...  Scores are computed for every slot
  // (no divergent branch around the epilogue); invalid slots count into bin
  // kNB, the row's padding slot, which no scan reads.
  auto scan_row = [&](int rl, int& nd) -> int {     // top-down cumulative search
    int cum = 0, bsel = 0;
    for (int bin = kNB - 1; bin >= 0; --bin) {
      const int c = H::count(&sh[rl * kHStride], bin);
      if (cum + c >= nd) { bsel = bin; break; }
      cum += c;
    }
    nd -= cum;
    return bsel;
  };
  auto zero_hist = [&]() {
    for (int i = tid; i < 16 * kHStride; i += kGroupThreads) sh[i] = 0u;
    __syncthreads();
  };

  if constexpr (kPhase == 2) {
    // histograms of phase 1 (same grid, so the same block index)
    const uint32_t* hsrc = sa.hist + (int64_t)blockIdx.x * (16 * kHStride);
    for (int i = tid; i < 16 * kHStride; i += kGroupThreads) sh[i] = hsrc[i];
  } else {
    zero_hist();
    {
      typename Mfma<T>::Op kb[Mfma<T>::kSteps], kn[Mfma<T>::kSteps];
      int t = wave;
      if (t < ntl) rgp.load_keys(t * 16, p.T, lane, kn);
      for (; t < ntl; t += kGroupWaves) {
#pragma unroll
        for (int s = 0; s < Mfma<T>::kSteps; ++s) kb[s] = kn[s];
        if (t + kGroupWaves < ntl) rgp.load_keys((t + kGroupWaves) * 16, p.T, lane, kn);
        floatx4 acc[kHi];
        rgp.mma(kb, acc);
        bool valid[4];
        slot_valid(t * 16 + lr, valid);
        floatx4 sc;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sc[e] = rgp.score(acc, e);
          const int bn = valid[e] ? bin_of(sc[e], inv_w[e]) : kNB;
          H::add(&sh[(4 * g + e) * kHStride], bn);
        }
        *reinterpret_cast<floatx4*>(wsg + t * kTile + lane * 4) = sc;
      }
    }
  }
  __syncthreads();
  if (kPhase != 1 && tid < 16 && st_mode[tid] == kActive) {
    int nd = st_need[tid];
    st_b1[tid] = scan_row(tid, nd);
    st_need[tid] = nd;
  }
  __syncthreads();
#pragma unroll
  for (int e = 0; e < 4; ++e) b1[e] = st_b1[4 * g + e];

  // Replay of the stored tiles in quads of 4 consecutive tiles (quad j =
  // tiles 4j .. 4j+3, one 64-key word pair of the mask).  Each wave takes
  // runs of kRun consecutive quads, runs round-robin over the waves, and
  // issues all loads of a run before using any: nothing loaded stays live
  // across an iteration, so the waits before each quad count only the loads
  // issued after it.  Tile indices past the last tile re-read the last one
  // (always in bounds) and every quad of a run is processed: a tile past the
  // diagonal has no valid slot (its columns lie after every row of the
  // group), so a quad j >= nquad contributes nothing, and fq must not store
  // for it.
  constexpr int kRun = 3;
  const int nquad = (ntl + 3) >> 2;
  auto load_quad = [&](int j, floatx4 (&v)[4]) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = min(4 * j + u, ntl - 1);
      v[u] = *reinterpret_cast<const floatx4*>(wsg + t * kTile + lane * 4);
    }
  };
  // f(quad, u, col, valid[4], score[4]) per tile, then fq(quad) per quad.
  auto replay = [&](auto&& f, auto&& fq) {
    for (int c = wave; kRun * c < nquad; c += kGroupWaves) {
      floatx4 qv[kRun][4];
#pragma unroll
      for (int r = 0; r < kRun; ++r) load_quad(kRun * c + r, qv[r]);
#pragma unroll
      for (int r = 0; r < kRun; ++r) {
        const int j = kRun * c + r;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int col = (4 * j + u) * 16 + lr;
          bool valid[4];
          slot_valid(col, valid);
          const float sc[4] = {qv[r][u][0], qv[r][u][1], qv[r][u][2], qv[r][u][3]};
          f(j, u, col, valid, sc);
        }
        fq(j);
      }
    }
  };

  if constexpr (kPhase == 1) {
    // ---- row variance (population, over the row's causal scores) --------------
    // Sums of d = s - c and d^2 with c = the row's mean estimated from its
    // histogram (bin centres; |mean - c| <= half a bin), so that the
    // difference S2/n - (S1/n)^2 keeps its precision.  Then the histograms
    // are saved for phase 2.
    __shared__ float st_shift[16];
    __shared__ float2 st_part[16 * kGroupWaves];
    if (wave == 0 && lr == 0) {
#pragma unroll
      for (int e = 0; e < 4; ++e) st_shift[4 * g + e] = inv_w[e];   // 1 / bin width
    }
    __syncthreads();
    {
      const int rl = (tid >> 4) & 15, part = tid & 15;   // threads 0..255: 16 per row, 32 bins each
      float m = 0.f;
      if (tid < 256)
        for (int bin = part * (kNB / 16); bin < (part + 1) * (kNB / 16); ++bin)
          m = __builtin_fmaf((float)H::count(&sh[rl * kHStride], bin), (float)bin + 0.5f, m);
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) m += __shfl_xor(m, o, 64);
      const int row = r0 + rl;
      const float iw = st_shift[rl];
      __syncthreads();
      if (tid < 256 && part == 0) st_shift[rl] = row < p.T ? m / ((float)(row + 1) * iw) : 0.f;
    }
    __syncthreads();
    float c[4], s1[4], s2[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      c[e] = st_shift[4 * g + e];
      s1[e] = 0.f;
      s2[e] = 0.f;
    }
    replay(
        [&](int, int, int, const bool (&valid)[4], const float (&sc)[4]) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float d = valid[e] ? sc[e] - c[e] : 0.f;
            s1[e] += d;
            s2[e] = __builtin_fmaf(d, d, s2[e]);
          }
        },
        [](int) {});
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        s1[e] += __shfl_xor(s1[e], o, 64);
        s2[e] += __shfl_xor(s2[e], o, 64);
      }
    if (lr == 0) {
#pragma unroll
      for (int e = 0; e < 4; ++e) st_part[(4 * g + e) * kGroupWaves + wave] = make_float2(s1[e], s2[e]);
    }
    __syncthreads();
    if (tid < 16 && r0 + tid < p.T) {
      float S1 = 0.f, S2 = 0.f;
#pragma unroll
      for (int w = 0; w < kGroupWaves; ++w) {
        S1 += st_part[tid * kGroupWaves + w].x;
        S2 += st_part[tid * kGroupWaves + w].y;
      }
      const float n = (float)(r0 + tid + 1);
      const float m1 = S1 / n;
      sa.row_var[(int64_t)b * p.T + r0 + tid] = fmaxf(S2 / n - m1 * m1, 0.f);
    }
    uint32_t* hdst = sa.hist + (int64_t)blockIdx.x * (16 * kHStride);
    for (int i = tid; i < 16 * kHStride; i += kGroupThreads) hdst[i] = sh[i];
    return;
  }

  // ---- pass 2: bins above b1 -> mask words; bin b1 -> candidates -------------
  // Candidates of row 4g+e found by this wave go to its own region of the
  // row's list in the workspace (kWCap slots), positions from a per-wave
  // count: no atomics.  Lane
  // 16g+e assembles row 4g+e's 64-bit mask word of each quad.
  int wc[4] = {0, 0, 0, 0};
  const uint32_t below = (1u << lr) - 1u;
  uint64_t word = 0;
  replay(
      [&](int, int u, int col, const bool (&valid)[4], const float (&sc)[4]) {
        uint64_t m[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int bn = bin_of(sc[e], inv_w[e]);
          m[e] = ballot64(valid[e] && bn > b1[e]);
          const bool is_cand = valid[e] && bn == b1[e];
          const uint64_t cm = ballot64(is_cand);
          if (cm) {
            const uint32_t gm = (uint32_t)(cm >> (16 * g)) & 0xffffu;
            const int pos = wc[e] + __popc(gm & below);
            if (is_cand && pos < kWCap)
              cand[(4 * g + e) * kCap + wave * kWCap + pos] = uint2{score_key(sc[e]), (uint32_t)col};
            wc[e] += __popc(gm);
          }
        }
        const uint64_t me = (lr & 2) ? ((lr & 1) ? m[3] : m[2]) : ((lr & 1) ? m[1] : m[0]);
        word |= ((me >> (16 * g)) & 0xffffull) << (16 * u);
      },
      [&](int j) {
        if (own_act && j < nquad) reinterpret_cast<uint64_t*>(bbase + (int64_t)own_row * b_st)[j] = word;
        word = 0;
      });
  if (lr == 0) {
#pragma unroll
    for (int e = 0; e < 4; ++e) sh_wcnt[(4 * g + e) * kGroupWaves + wave] = (uint32_t)wc[e];
  }
  // The resolve's atomics and candidate reads below come from waves of this
  // block only: the barrier (a workgroup-scope release/acquire) orders the
  // mask and candidate stores above before them.  A device-scope fence here
  // would write back the whole L2.
  __syncthreads();

  // ---- resolve: wave w takes rows kRW*w .. kRW*w + kRW-1 ----------------------
  // Candidate slot i*64 + lane lies in region i/2 at position (i%2)*64 + lane.
  constexpr int kRW = 16 / kGroupWaves;
  for (int q = 0; q < kRW; ++q) {
    const int rl = kRW * wave + q;
    if (st_mode[rl] != kActive) continue;
    int nw[kGroupWaves];
    bool ovf = false;
#pragma unroll
    for (int w = 0; w < kGroupWaves; ++w) {
      nw[w] = (int)sh_wcnt[rl * kGroupWaves + w];
      ovf |= nw[w] > kWCap;
    }
    if (ovf) {
      if (lane == 0) { st_mode[rl] = kOverflow; st_any[1] = 1; }
      continue;
    }
    // The row's n candidates, compacted: candidate j (in the regions' order)
    // goes to slot j / 64, lane j % 64, so the radix passes below ballot
    // ceil(n / 64) slots instead of one per occupied region half.
    constexpr int kSlots = kCap / 64;
    int start[kGroupWaves];
    int n = 0;
#pragma unroll
    for (int w = 0; w < kGroupWaves; ++w) { start[w] = n; n += nw[w]; }
    uint32_t cv[kSlots], ci[kSlots];
    bool cvalid[kSlots], used[kSlots];
    uint32_t kor = 0u, kand = ~0u;
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      const int j = i * 64 + lane;
      used[i] = i * 64 < n;
      cvalid[i] = j < n;
      int w = 0;
#pragma unroll
      for (int ww = 1; ww < kGroupWaves; ++ww) w += j >= start[ww] ? 1 : 0;
      const uint2 cd = cvalid[i] ? cand[rl * kCap + w * kWCap + (j - start[w])] : uint2{0u, 0u};
      cv[i] = cd.x;
      ci[i] = cd.y;
      if (cvalid[i]) { kor |= cv[i]; kand &= cv[i]; }
    }
    // Bits on which every candidate agrees are part of theta; the radix
    // select starts at the highest bit on which they differ.
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      kor |= (uint32_t)__shfl_xor((int)kor, o, 64);
      kand &= (uint32_t)__shfl_xor((int)kand, o, 64);
    }
    int k = st_need[rl];
    const uint32_t diff = kor ^ kand;
    const int top = diff ? 31 - __builtin_clz(diff) : -1;
    uint32_t pmask = top >= 31 ? 0u : ~0u << (top + 1);
    uint32_t prefix = kand & pmask;
    for (int bit = top; bit >= 0; --bit) {
      const uint32_t tm = pmask | (1u << bit), tv = prefix | (1u << bit);
      int c = 0;
#pragma unroll
      for (int i = 0; i < kSlots; ++i)
        if (used[i]) c += __popcll(ballot64(cvalid[i] && (cv[i] & tm) == tv));
      if (c >= k) prefix = tv; else k -= c;
      pmask = tm;
    }
    // winners: key > theta, or key == theta among the k lowest indices of the
    // ties (all of them when there are at most k)
    int ties = 0;
#pragma unroll
    for (int i = 0; i < kSlots; ++i)
      if (used[i]) ties += __popcll(ballot64(cvalid[i] && cv[i] == prefix));
    const int row = r0 + rl;
    uint32_t* brow = bbase + (int64_t)row * b_st;
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      if (!used[i] || !cvalid[i]) continue;
      bool win = cv[i] > prefix;
      if (cv[i] == prefix) {
        if (ties <= k) {
          win = true;
        } else {
          int rank = 0;
          for (int w = 0; w < kGroupWaves; ++w)
            for (int o = 0; o < nw[w]; ++o) {
              const uint2 cd = cand[rl * kCap + w * kWCap + o];
              rank += (cd.x == prefix && cd.y < ci[i]) ? 1 : 0;
            }
          win = rank < k;
        }
      }
      if (win) atomicOr(&brow[ci[i] >> 5], 1u << (ci[i] & 31));
    }
  }
  __syncthreads();
  if (!st_any[1]) return;

  // ---- overflow rows: radix passes over the stored scores of bin b1 -----------
  if (tid < 16 && st_mode[tid] == kOverflow) st_key[tid] = 0u;
#pragma unroll
  for (int e = 0; e < 4; ++e) act[e] = st_mode[4 * g + e] == kOverflow;
  for (int level = 0; level < 4; ++level) {
    uint32_t pre[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) pre[e] = st_key[4 * g + e];
    const int hi_shift = 32 - 8 * level, lo_shift = 24 - 8 * level;
    zero_hist();
    replay(
        [&](int, int, int, const bool (&valid)[4], const float (&sc)[4]) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (valid[e] && bin_of(sc[e], inv_w[e]) == b1[e]) {
              const uint32_t key = score_key(sc[e]);
              if (level == 0 || (key >> hi_shift) == pre[e])
                atomicAdd(&sh[(4 * g + e) * kHStride + ((key >> lo_shift) & 255u)], 1u);
            }
          }
        },
        [](int) {});
    __syncthreads();
    if (tid < 16 && st_mode[tid] == kOverflow) {
      int cum = 0, d = 0, nd = st_need[tid];
      for (int bin = 255; bin >= 0; --bin) {
        const int c = (int)sh[tid * kHStride + bin];
        if (cum + c >= nd) { d = bin; break; }
        cum += c;
      }
      st_need[tid] = nd - cum;
      st_key[tid] = (st_key[tid] << 8) | (uint32_t)d;
    }
    __syncthreads();
  }
  // wave 0 marks the winners of the overflow rows in key order (tie ranks need
  // order); every wave's stored tiles are visible after the barriers above
  if (wave == 0) {
    uint32_t theta[4];
    int tie_need[4], tie_seen[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      theta[e] = st_key[4 * g + e];
      tie_need[e] = st_need[4 * g + e];
      tie_seen[e] = 0;
    }
    const uint64_t gmask = 0xffffull << (16 * g);
    for (int t = 0; t < ntl; ++t) {
      const floatx4 v = *reinterpret_cast<const floatx4*>(wsg + t * kTile + lane * 4);
      const int col = t * 16 + lr;
      bool valid[4];
      slot_valid(col, valid);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = r0 + 4 * g + e;
        const bool inbin = valid[e] && bin_of(v[e], inv_w[e]) == b1[e];
        const uint32_t key = score_key(v[e]);
        const bool tie = inbin && key == theta[e];
        const uint64_t tmask = ballot64(tie) & gmask;
        const int trank = tie_seen[e] + count_below(tmask);
        tie_seen[e] += __popcll(tmask);
        if (inbin && (key > theta[e] || (tie && trank < tie_need[e])))
          atomicOr(&bbase[(int64_t)row * b_st + (col >> 5)], 1u << (col & 31));
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Bitmask -> ascending indices + count, one 256-thread block per row.  Row
// t of width k_eff holds its n = min(t+1, k_t) selected keys ascending (k_t
// = k_rows[row] capped at k_eff, or k_eff when k_rows is null), then t+1,
// t+2, ... up to entry k_t - 1 (the lowest-index invalid entries, as the
// selector orders them; entries below k_t past n exist only when t+1 < k_t,
// so these stay below k_t <= T), then index 0 in entries k_t .. k_eff - 1
// (like the adaptive standalone selector's entries past k_t).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void bits_to_indices_kernel(const uint32_t* __restrict__ bits, int64_t b_sb,
                                                              int64_t b_st, int T, int W, int k_eff,
                                                              const int32_t* __restrict__ k_rows,
                                                              int32_t* __restrict__ idx_out,
                                                              int32_t* __restrict__ count_out) {
  __shared__ int wave_tot[4];
  const int row = blockIdx.x;
  const int b = row / T, t = row % T;
  const uint32_t* brow = bits + b * b_sb + (int64_t)t * b_st;
  int32_t* orow = idx_out + (int64_t)row * k_eff;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int per = (W + 255) / 256;       // contiguous words per thread
  const int w0 = min(W, tid * per), w1 = min(W, w0 + per);
  int cnt = 0;
  for (int wd = w0; wd < w1; ++wd) cnt += __popc(brow[wd]);
  // exclusive prefix over the block
  int incl = cnt;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(incl, off, 64);
    if (lane >= off) incl += y;
  }
  if (lane == 63) wave_tot[wave] = incl;
  __syncthreads();
  int base = incl - cnt, total = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    if (w < wave) base += wave_tot[w];
    total += wave_tot[w];
  }
  int pos = base;
  for (int wd = w0; wd < w1; ++wd) {
    uint32_t m = brow[wd];
    while (m) {
      const int bit = __ffs(m) - 1;
      m &= m - 1;
      if (pos < k_eff) orow[pos] = wd * 32 + bit;
      ++pos;
    }
  }
  const int n = min(total, k_eff);
  const int k_row = k_rows ? min(k_rows[row], k_eff) : k_eff;
  for (int i = n + tid; i < k_eff; i += 256) orow[i] = i < k_row ? t + 1 + (i - n) : 0;
  if (tid == 0) count_out[row] = n;
}

// ---------------------------------------------------------------------------
// Variance-based adaptive k (gsa_explained.ipynb:577-592): with avg = the mean
// of every row's variance over all B*T rows (clamped to >= 1e-6),
//   k_t = clamp(floor(k_base * avg / max(var_t, 1e-6)), k_min, k_max),
// then capped at k_cap = min(k_max, T).  One block; the sum runs in double in
// a fixed order (deterministic), the per-row rule in fp32 in the formula's
// order (k_base * avg, then the correctly rounded division).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void adaptive_k_kernel(const float* __restrict__ var, int n, int k_base,
                                                          int k_min, int k_max, int k_cap,
                                                          int* __restrict__ k_rows) {
  __shared__ double part[16];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  double sum = 0.0;
  for (int i = tid; i < n; i += 1024) sum += (double)var[i];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
  if (lane == 0) part[wave] = sum;
  __syncthreads();
  double tot = 0.0;
#pragma unroll
  for (int w = 0; w < 16; ++w) tot += part[w];
  const float avg = fmaxf((float)(tot / (double)n), 1e-6f);
  const float num = (float)k_base * avg;
  for (int i = tid; i < n; i += 1024) {
    const float r = floorf(num / fmaxf(var[i], 1e-6f));
    const float c = fminf(fmaxf(r, (float)k_min), (float)k_max);
    k_rows[i] = min((int)c, k_cap);
  }
}

}  // namespace gsa

// ---------------------------------------------------------------------------
// Host entry points
// ---------------------------------------------------------------------------
using namespace gsa_host;

static int check_indexer_args(const void* q, int64_t q_sb, int64_t q_st, const void* k, int64_t k_sb,
                              int64_t k_st, const void* w, const float* bias, int B, int T, int Hi,
                              int di, int dtype) {
  if (!q || !k || !w || !bias) return GSA_ERR_NULL;
  if (dtype_size(dtype) == 0) return GSA_ERR_DTYPE;
  if (B < 1 || T < 1 || Hi != gsa::kHi || di != gsa::kDi) return GSA_ERR_SHAPE;
  if (!vec_ok(q, q_sb, q_st, dtype) || !vec_ok(k, k_sb, k_st, dtype)) return GSA_ERR_ALIGN;
  if (!aligned(w, dtype_size(dtype)) || !aligned(bias, 4)) return GSA_ERR_ALIGN;
  return GSA_OK;
}

static gsa::IdxArgs make_idx_args(const void* q, int64_t q_sb, int64_t q_st, const void* k, int64_t k_sb,
                                  int64_t k_st, const void* w, int64_t w_sb, int64_t w_st,
                                  const float* bias, float scale, int B, int T) {
  gsa::IdxArgs a;
  a.q = q; a.q_sb = q_sb; a.q_st = q_st;
  a.k = k; a.k_sb = k_sb; a.k_st = k_st;
  a.w = w; a.w_sb = w_sb; a.w_st = w_st;
  a.bias = bias;
  a.scale_l2 = -scale * gsa::kLog2e;
  a.B = B; a.T = T;
  return a;
}

extern "C" int gsa_indexer_scores(const void* q_idx, int64_t q_sb, int64_t q_st,
                                  const void* k_idx, int64_t k_sb, int64_t k_st,
                                  const void* w, int64_t w_sb, int64_t w_st,
                                  const float* bias, float scale,
                                  int B, int T, int Hi, int di, int causal, int dtype,
                                  float* scores, int64_t s_sb, int64_t s_st,
                                  void* stream) {
  int st = check_indexer_args(q_idx, q_sb, q_st, k_idx, k_sb, k_st, w, bias, B, T, Hi, di, dtype);
  if (st) return st;
  if (!scores) return GSA_ERR_NULL;
  if (!aligned(scores, 4)) return GSA_ERR_ALIGN;
  gsa::IdxArgs a = make_idx_args(q_idx, q_sb, q_st, k_idx, k_sb, k_st, w, w_sb, w_st, bias, scale, B, T);
  const int ngroups = (T + 15) / 16;
  const int waves = B * ngroups;
  dim3 grid((waves + 3) / 4), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == GSA_DTYPE_BF16)
    hipLaunchKernelGGL(gsa::indexer_scores_kernel<uint16_t>, grid, block, 0, s, a, causal, scores, s_sb, s_st);
  else
    hipLaunchKernelGGL(gsa::indexer_scores_kernel<float>, grid, block, 0, s, a, causal, scores, s_sb, s_st);
  return launch_status();
}

// One launch of the fused selector in phase kPhase; the 16-bit histogram
// counts are exact while a row has at most 65535 keys.
template <int kPhase>
static void launch_bits(const gsa::IdxArgs& a, const gsa::SelArgs& sa, int dtype, uint32_t* bits,
                        int64_t b_sb, int64_t b_st, float* wsf, uint2* wsc, hipStream_t s) {
  const bool packed = a.T <= 65535;
  const dim3 grid(a.B * ((a.T + 15) / 16)), block(gsa::kGroupThreads);
  if (dtype == GSA_DTYPE_BF16) {
    if (packed)
      hipLaunchKernelGGL((gsa::indexer_bits_kernel<uint16_t, true, kPhase>), grid, block, 0, s, a, sa, bits, b_sb, b_st, wsf, wsc);
    else
      hipLaunchKernelGGL((gsa::indexer_bits_kernel<uint16_t, false, kPhase>), grid, block, 0, s, a, sa, bits, b_sb, b_st, wsf, wsc);
  } else {
    if (packed)
      hipLaunchKernelGGL((gsa::indexer_bits_kernel<float, true, kPhase>), grid, block, 0, s, a, sa, bits, b_sb, b_st, wsf, wsc);
    else
      hipLaunchKernelGGL((gsa::indexer_bits_kernel<float, false, kPhase>), grid, block, 0, s, a, sa, bits, b_sb, b_st, wsf, wsc);
  }
}

// Score tiles (1 KiB per causal 16x16 tile), then the candidate lists
// (16 rows x kCap (key, index) pairs per 16-row group).
static size_t score_ws_bytes(int B, int T) {
  const size_t g = (size_t)((T + 15) / 16);
  return (size_t)B * (g * (g + 1) / 2) * gsa::kTile * sizeof(float);
}

extern "C" size_t gsa_indexer_select_workspace_bytes(int B, int T) {
  if (B < 1 || T < 1) return 0;
  const size_t g = (size_t)((T + 15) / 16);
  return score_ws_bytes(B, T) + (size_t)B * g * 16 * gsa::kCap * sizeof(uint2);
}

int gsa_host::launch_adaptive_k(const float* var, int n, int k_base, int k_min, int k_max, int k_cap,
                                int32_t* k_rows, hipStream_t stream) {
  hipLaunchKernelGGL(gsa::adaptive_k_kernel, dim3(1), dim3(1024), 0, stream, var, n, k_base, k_min, k_max, k_cap,
                     k_rows);
  return launch_status();
}

// Argument checks shared by the fixed and the adaptive selector.
static int check_select_args(const void* q_idx, int64_t q_sb, int64_t q_st, const void* k_idx, int64_t k_sb,
                             int64_t k_st, const void* w, const float* bias, int B, int T, int Hi, int di,
                             int dtype, const uint32_t* bits, int64_t b_sb, int64_t b_st,
                             const int32_t* idx_out, const int32_t* count_out, const void* ws) {
  int st = check_indexer_args(q_idx, q_sb, q_st, k_idx, k_sb, k_st, w, bias, B, T, Hi, di, dtype);
  if (st) return st;
  if (!bits || !ws) return GSA_ERR_NULL;
  if ((idx_out == nullptr) != (count_out == nullptr)) return GSA_ERR_NULL;
  const int W = 2 * ((T + 63) / 64);
  if (b_st < W || (B > 1 && b_sb < (int64_t)T * b_st)) return GSA_ERR_SHAPE;
  if (!aligned(bits, 8) || (b_st % 2) || (b_sb % 2)) return GSA_ERR_ALIGN;
  if (idx_out && (!aligned(idx_out, 4) || !aligned(count_out, 4))) return GSA_ERR_ALIGN;
  if ((int64_t)B * T > 0x7fffffffLL) return GSA_ERR_SHAPE;
  if (!aligned(ws, 16)) return GSA_ERR_ALIGN;
  return GSA_OK;
}

extern "C" int gsa_indexer_select(const void* q_idx, int64_t q_sb, int64_t q_st,
                                  const void* k_idx, int64_t k_sb, int64_t k_st,
                                  const void* w, int64_t w_sb, int64_t w_st,
                                  const float* bias, float scale,
                                  int B, int T, int Hi, int di, int k_eff, int dtype,
                                  uint32_t* bits, int64_t b_sb, int64_t b_st,
                                  int32_t* idx_out, int32_t* count_out,
                                  void* ws, size_t ws_bytes, void* stream) {
  int st = check_select_args(q_idx, q_sb, q_st, k_idx, k_sb, k_st, w, bias, B, T, Hi, di, dtype, bits, b_sb,
                             b_st, idx_out, count_out, ws);
  if (st) return st;
  if (k_eff < 1 || k_eff > T) return GSA_ERR_K;
  if (ws_bytes < gsa_indexer_select_workspace_bytes(B, T)) return GSA_ERR_SHAPE;
  gsa::IdxArgs a = make_idx_args(q_idx, q_sb, q_st, k_idx, k_sb, k_st, w, w_sb, w_st, bias, scale, B, T);
  hipStream_t s = static_cast<hipStream_t>(stream);
  float* wsf = static_cast<float*>(ws);
  uint2* wsc = reinterpret_cast<uint2*>(static_cast<char*>(ws) + score_ws_bytes(B, T));
  gsa::SelArgs sa{k_eff, nullptr, nullptr, nullptr};
  launch_bits<0>(a, sa, dtype, bits, b_sb, b_st, wsf, wsc, s);
  st = launch_status();
  if (st || !idx_out) return st;
  const int W = 2 * ((T + 63) / 64);
  hipLaunchKernelGGL(gsa::bits_to_indices_kernel, dim3(B * T), dim3(256), 0, s, bits, b_sb, b_st, T, W, k_eff,
                     nullptr, idx_out, count_out);
  return launch_status();
}

// Adaptive workspace: the fixed selector's, then the phase-1 histograms (16
// rows x Hist::kStride words per 16-row group), then the per-row variances
// and k values ([B*T] each, used when the caller does not take them).
static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

static size_t hist_ws_bytes(int B, int T) {
  const size_t g = (size_t)((T + 15) / 16);
  const size_t stride = T <= 65535 ? gsa::Hist<true>::kStride : gsa::Hist<false>::kStride;
  return (size_t)B * g * 16 * stride * sizeof(uint32_t);
}

extern "C" size_t gsa_indexer_select_adaptive_workspace_bytes(int B, int T) {
  if (B < 1 || T < 1) return 0;
  return align256(gsa_indexer_select_workspace_bytes(B, T)) + align256(hist_ws_bytes(B, T)) +
         2 * align256((size_t)B * T * sizeof(float));
}

extern "C" int gsa_indexer_select_adaptive(const void* q_idx, int64_t q_sb, int64_t q_st,
                                           const void* k_idx, int64_t k_sb, int64_t k_st,
                                           const void* w, int64_t w_sb, int64_t w_st,
                                           const float* bias, float scale,
                                           int B, int T, int Hi, int di,
                                           int k_base, int k_min, int k_max, int dtype,
                                           uint32_t* bits, int64_t b_sb, int64_t b_st,
                                           int32_t* idx_out, int32_t* count_out,
                                           int32_t* k_out, float* var_out,
                                           void* ws, size_t ws_bytes, void* stream) {
  int st = check_select_args(q_idx, q_sb, q_st, k_idx, k_sb, k_st, w, bias, B, T, Hi, di, dtype, bits, b_sb,
                             b_st, idx_out, count_out, ws);
  if (st) return st;
  if (k_base < 1 || k_min < 1 || k_max < k_min) return GSA_ERR_K;
  if ((k_out && !aligned(k_out, 4)) || (var_out && !aligned(var_out, 4))) return GSA_ERR_ALIGN;
  if (ws_bytes < gsa_indexer_select_adaptive_workspace_bytes(B, T)) return GSA_ERR_SHAPE;
  const int k_cap = k_max < T ? k_max : T;
  gsa::IdxArgs a = make_idx_args(q_idx, q_sb, q_st, k_idx, k_sb, k_st, w, w_sb, w_st, bias, scale, B, T);
  hipStream_t s = static_cast<hipStream_t>(stream);
  char* base = static_cast<char*>(ws);
  float* wsf = reinterpret_cast<float*>(base);
  uint2* wsc = reinterpret_cast<uint2*>(base + score_ws_bytes(B, T));
  size_t off = align256(gsa_indexer_select_workspace_bytes(B, T));
  uint32_t* hist = reinterpret_cast<uint32_t*>(base + off);
  off += align256(hist_ws_bytes(B, T));
  float* var = var_out ? var_out : reinterpret_cast<float*>(base + off);
  off += align256((size_t)B * T * sizeof(float));
  int32_t* krow = k_out ? k_out : reinterpret_cast<int32_t*>(base + off);

  launch_bits<1>(a, gsa::SelArgs{0, nullptr, var, hist}, dtype, bits, b_sb, b_st, wsf, wsc, s);
  if ((st = launch_status())) return st;
  if ((st = launch_adaptive_k(var, B * T, k_base, k_min, k_max, k_cap, krow, s))) return st;
  launch_bits<2>(a, gsa::SelArgs{0, krow, nullptr, hist}, dtype, bits, b_sb, b_st, wsf, wsc, s);
  st = launch_status();
  if (st || !idx_out) return st;
  const int W = 2 * ((T + 63) / 64);
  hipLaunchKernelGGL(gsa::bits_to_indices_kernel, dim3(B * T), dim3(256), 0, s, bits, b_sb, b_st, T, W, k_cap,
                     krow, idx_out, count_out);
  return launch_status();
}
