// Gated lightning indexer on gfx950 MFMA, and its fused exact top-k select.
//
//   S[b,i,j] = sum_h sigmoid(w[b,i,h]) * sigmoid(scale*<q[b,i,h,:], k[b,j,:]> + bias[h])
//
// (semantics of gsa_triton/gsa_ref.py:97-126).  Both kernels below share one
// score routine -- the same MFMA sequence and the same epilogue instructions
// -- so a score is bit-identical wherever it is computed; the fused selector
// relies on that when it recomputes scores pass after pass.
//
// Tiling: one wave owns 16 query rows.  The product is taken transposed,
// D = K Q^T: the MFMA A operand is a tile of 16 keys (streamed), the B
// operand the wave's 16 query rows (4 heads x 64 dims, in registers for the
// whole kernel):
//   bf16: v_mfma_f32_16x16x32_bf16, 2 k-steps per head  (8 MFMA per tile)
//   fp32: v_mfma_f32_16x16x4_f32,  16 k-steps per head (64 MFMA per tile)
// Output layout of a 16x16 block: lane l holds rows 4*(l/16)+e (e = 0..3)
// of column l%16, i.e. query row r0 + l%16 against the four consecutive keys
// j0 + 4*(l/16) + e.  Every per-row quantity is therefore lane-local.
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
  // the same element group from a byte address (row start + group_bytes(g))
  __device__ static uint32_t group_bytes(int g) { return (uint32_t)g * 16u; }
  __device__ static Op load_at(const char* p, int s) { return *reinterpret_cast<const bf16x8*>(p + s * 64); }
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
  __device__ static uint32_t group_bytes(int g) { return (uint32_t)g * 4u; }
  __device__ static Op load_at(const char* p, int s) { return *reinterpret_cast<const float*>(p + s * 16); }
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

// Per-lane state of one wave's 16-row group: lane l works for query row
// r0 + l%16.
template <typename T>
struct RowGroup {
  typename Mfma<T>::Op qb[kHi][Mfma<T>::kSteps];  // B operand: query row r0 + lane%16
  float a[kHi];                                   // sigmoid(w) of the lane's row
  float c01, c23;                                 // a0 + a1, a2 + a3
  float bias_l2[kHi];                             // -bias[h] * log2(e)
  float scale_l2;                                 // -scale * log2(e)
  const char* kbase;                              // k_idx of this batch
  int64_t kst_bytes;                              // its row stride in bytes
  uint32_t koff;                                  // the lane's byte offset in a key tile

  __device__ void init(const IdxArgs& p, int b, int r0, int lane) {
    const int g = lane >> 4, lr = lane & 15;
    const int row = min(r0 + lr, p.T - 1);
    const T* qrp = static_cast<const T*>(p.q) + b * p.q_sb + (int64_t)row * p.q_st;
#pragma unroll
    for (int h = 0; h < kHi; ++h)
#pragma unroll
      for (int s = 0; s < Mfma<T>::kSteps; ++s) qb[h][s] = Mfma<T>::load(qrp, h * kDi, s, g);
    const T* wrp = static_cast<const T*>(p.w) + b * p.w_sb + (int64_t)row * p.w_st;
#pragma unroll
    for (int h = 0; h < kHi; ++h) {
      const T wv = wrp[h];
      float wf;
      if constexpr (Elem<T>::kBf16) wf = __uint_as_float((uint32_t)wv << 16);
      else wf = wv;
      a[h] = sigmoidf_fast(wf);
    }
    c01 = a[0] + a[1];
    c23 = a[2] + a[3];
    kbase = reinterpret_cast<const char*>(static_cast<const T*>(p.k) + b * p.k_sb);
    kst_bytes = p.k_st * (int64_t)sizeof(T);
    koff = (uint32_t)((lane & 15) * kst_bytes) + Mfma<T>::group_bytes(g);
#pragma unroll
    for (int h = 0; h < kHi; ++h) bias_l2[h] = -p.bias[h] * kLog2e;
    scale_l2 = p.scale_l2;
  }

  // A operand of key tile [j0, j0+16): key j0 + lane%16, clamped to a valid
  // row.  The tile's base is uniform (scalar arithmetic) and each lane adds
  // its 32-bit offset; only a tile that reaches past row T-1 (the last one)
  // computes clamped offsets.  (The host keeps 16 rows of k below 2^31 bytes.)
  __device__ void load_keys(int j0, int T_, int lane, typename Mfma<T>::Op (&kb)[Mfma<T>::kSteps]) const {
    const char* tb = kbase + (int64_t)j0 * kst_bytes;
    uint32_t off = koff;
    if (j0 + 16 > T_) off = (uint32_t)(min(lane & 15, T_ - 1 - j0) * kst_bytes) + Mfma<T>::group_bytes(lane >> 4);
#pragma unroll
    for (int s = 0; s < Mfma<T>::kSteps; ++s) kb[s] = Mfma<T>::load_at(tb + off, s);
  }

  __device__ void mma(const typename Mfma<T>::Op (&kb)[Mfma<T>::kSteps], floatx4 (&acc)[kHi]) const {
#pragma unroll
    for (int h = 0; h < kHi; ++h) {
      floatx4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < Mfma<T>::kSteps; ++s) c = Mfma<T>::mma(kb[s], qb[h][s], c);
      acc[h] = c;
    }
  }

  // Fused epilogue for slot e: sum_h a_h * sigmoid(scale*dot_h + bias_h).
  // With x_h = 2^(-(scale*dot_h + bias_h) log2 e), sigmoid = 1/(1 + x_h), and
  // the four terms are summed over one common denominator,
  //   a0/(1+x0) + a1/(1+x1) = (a0 + a1 + a0 x1 + a1 x0) / ((1+x0)(1+x1)),
  // the two pairs likewise: 4 exp2 and 1 reciprocal instead of 4 + 4.  Every
  // term is positive, so nothing cancels; the result is within a few fp32
  // ulps of the per-head form.  When the common denominator leaves the
  // range where numerator and denominator are finite (some x_h beyond about
  // 2^31, or a non-finite input), the per-head form runs instead.
  __device__ float score(const floatx4 (&acc)[kHi], int e) const {
    float x[kHi];
#pragma unroll
    for (int h = 0; h < kHi; ++h) x[h] = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[h][e], scale_l2, bias_l2[h]));
    const float u0 = 1.0f + x[0], u2 = 1.0f + x[2];
    const float d01 = __builtin_fmaf(u0, x[1], u0);     // (1+x0)(1+x1)
    const float d23 = __builtin_fmaf(u2, x[3], u2);
    const float n01 = __builtin_fmaf(a[1], x[0], __builtin_fmaf(a[0], x[1], c01));
    const float n23 = __builtin_fmaf(a[3], x[2], __builtin_fmaf(a[2], x[3], c23));
    const float den = d01 * d23;
    const float num = __builtin_fmaf(n01, d23, n23 * d01);
    float s = num * __builtin_amdgcn_rcpf(den);
    if (!(den < 0x1p124f)) s = per_head(x);   // also NaN
    return s;
  }
  __device__ float per_head(const float (&x)[kHi]) const {
    float s = a[0] * __builtin_amdgcn_rcpf(1.0f + x[0]);
#pragma unroll
    for (int h = 1; h < kHi; ++h) s = __builtin_fmaf(a[h], __builtin_amdgcn_rcpf(1.0f + x[h]), s);
    return s;
  }
  // score() of the four slots of a tile, bit for bit, with one range test
  // for the tile: the sum of the four (positive) denominators is below
  // 2^124 only if each is, and it is NaN if any is.
  __device__ void score4(const floatx4 (&acc)[kHi], float (&sc)[4]) const {
    float x[4][kHi], den[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
#pragma unroll
      for (int h = 0; h < kHi; ++h)
        x[e][h] = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[h][e], scale_l2, bias_l2[h]));
      const float u0 = 1.0f + x[e][0], u2 = 1.0f + x[e][2];
      const float d01 = __builtin_fmaf(u0, x[e][1], u0);
      const float d23 = __builtin_fmaf(u2, x[e][3], u2);
      const float n01 = __builtin_fmaf(a[1], x[e][0], __builtin_fmaf(a[0], x[e][1], c01));
      const float n23 = __builtin_fmaf(a[3], x[e][2], __builtin_fmaf(a[2], x[e][3], c23));
      den[e] = d01 * d23;
      const float num = __builtin_fmaf(n01, d23, n23 * d01);
      sc[e] = num * __builtin_amdgcn_rcpf(den[e]);
    }
    if (!((den[0] + den[1]) + (den[2] + den[3]) < 0x1p124f)) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (!(den[e] < 0x1p124f)) sc[e] = per_head(x[e]);
    }
  }
};

// ---------------------------------------------------------------------------
// Full score matrix (the fused_gated_indexer API).  4 waves per block, one
// 16-row group per wave; causal tiles above the diagonal are filled with -inf
// without computing them.  A lane writes its row's four consecutive keys of
// a tile with one 16-byte store when `vec` (scores, s_sb and s_st allow it).
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void indexer_scores_kernel(IdxArgs p, int causal, float* S,
                                                             int64_t s_sb, int64_t s_st, int vec) {
  const int lane = threadIdx.x & 63;
  const int ngroups = (p.T + 15) >> 4;
  const int wv = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wv >= p.B * ngroups) return;
  const int b = wv / ngroups;
  const int r0 = (wv % ngroups) * 16;
  const int g = lane >> 4, lr = lane & 15;
  const int row = r0 + lr;

  RowGroup<T> rg;
  rg.init(p, b, r0, lane);
  float* srow = S + b * s_sb + (int64_t)min(row, p.T - 1) * s_st;
  auto put = [&](int col0, const float (&v)[4]) {
    if (row >= p.T) return;
    if (vec && col0 + 3 < p.T) {
      *reinterpret_cast<floatx4*>(srow + col0) = floatx4{v[0], v[1], v[2], v[3]};
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (col0 + e < p.T) srow[col0 + e] = v[e];
    }
  };

  const int jend = causal ? min(p.T, r0 + 16) : p.T;
  typename Mfma<T>::Op kb[Mfma<T>::kSteps], kn[Mfma<T>::kSteps];
  rg.load_keys(0, p.T, lane, kn);
  for (int j0 = 0; j0 < jend; j0 += 16) {
#pragma unroll
    for (int s = 0; s < Mfma<T>::kSteps; ++s) kb[s] = kn[s];
    if (j0 + 16 < jend) rg.load_keys(j0 + 16, p.T, lane, kn);
    floatx4 acc[kHi];
    rg.mma(kb, acc);
    const int col0 = j0 + 4 * g;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = (causal && col0 + e > row) ? -__builtin_inff() : rg.score(acc, e);
    put(col0, v);
  }
  const float ninf[4] = {-__builtin_inff(), -__builtin_inff(), -__builtin_inff(), -__builtin_inff()};
  for (int j0 = ((jend + 15) >> 4) << 4; j0 < p.T; j0 += 16) put(j0 + 4 * g, ninf);
}
// ---------------------------------------------------------------------------
// Fused indexer + exact top-k.
//
// Output: the selection as a bitmask, bits[b][t] bit j set iff key j is one
// of row t's selected keys (W = 2*ceil(T/64) uint32 words per row; words past
// row t's causal range are zero).  One 1024-thread block (16 waves) per
// 16-row group, heaviest groups first; the waves share the group's causal
// 16-key tiles.  Rows with t+1 <= k select every causal key.  For the
// others, no score is ever stored:
//   sample  exact scores of every fourth tile (the first of each 64-key
//           quad) -> a value-linear histogram per row, bin = floor(s * NB /
//           sum_h sigmoid(w_h)) -> a band [lo, hi] around the k-th largest
//           score: the sample ranks k*n_s/n -+ (z*sigma + 2), sigma the
//           standard deviation of the sample count above a population
//           quantile (hypergeometric), z = 5;
//   main    exact scores of every tile: s > hi (or NaN) is a sure winner and
//           goes straight into the row's 64-bit mask word (one store per
//           quad); lo <= s <= hi is a candidate, kept as (score bits, key
//           index) in the LDS list of the lane that computed it, or in the
//           row's overflow list once that one is full; below lo is dropped;
//   resolve a row is proven exact when n_sure <= k <= n_sure + n_cand (the
//           k best in (score desc, index asc) order are then the sure ones and
//           the first k - n_sure candidates in that order): one wave per row
//           radix-selects the threshold key among the candidates with 8-bit
//           digit histograms, the first digit spanning the candidates' own
//           key range, breaks ties at it by lowest index, and ORs the winners
//           into the mask;
//   fallback  a row that fails the check (the band missed -- about 6e-7 per
//           row on independent scores -- its list overflowed, or degenerate
//           scores put the whole row in the band) is selected by an exact
//           radix select over recomputed scores: four 8-bit digit passes of
//           the score key, two digit passes of the index among ties at the
//           threshold, then one marking pass that rewrites the row's words.
//
// Memory order.  On gfx950 vector loads and stores share one completion
// counter, which the compiler's waits count in issue order: a wait for a
// prefetched key tile also waits for any store issued after it on some path
// that the compiler cannot count.  So the tile loops issue a fixed number of
// vector memory instructions per tile -- the next tile's key loads, issued
// before this tile's are consumed, unconditional (clamped to the last tile)
// and into the other of two register buffers, and one unconditional mask-word
// store per quad (lanes with nothing to write store to a sink slot) --
// and the candidate lists, the only data-dependent writes, live in LDS.
// ---------------------------------------------------------------------------
constexpr int kNB = 1024;                 // sample histogram bins per row
constexpr int kHStride = kNB / 2 + 1;     // words per row: 16-bit counts, two per word (+1: bank spread)
constexpr int kGroupWaves = 16;           // waves per 16-row group
constexpr int kGroupThreads = 64 * kGroupWaves;
// Candidate lists.  Each row has 64 writers -- its four lanes in each of the
// 16 waves -- and every writer a private list of kPrivCap slots; a writer
// whose list is full spills into the row's overflow list (kOvfCap slots,
// filled through an atomic counter).  A row holds 64 * 12 + 640 = 1408
// candidates at most (the band of a row of 16384 keys at k = 4096 holds about
// 1000); a row with more takes the fallback.  The lists fill the LDS a block
// may use: 138 KiB of pool + 19 KiB of fixed arrays.
constexpr int kPrivCap = 12;
constexpr int kPrivSlots = kPrivCap + 1;          // + one trash slot per writer (stores of non-candidates)
constexpr int kOvfCap = 640;
constexpr int kPrivWords = 16 * kPrivSlots * 64; // private slots of the 16 rows: [row][slot][writer]
constexpr int kKeyWords = kPrivWords + 16 * kOvfCap;
constexpr float kBandZ = 5.f;             // band half-width in standard deviations of the sample rank
constexpr int kFbStride = 512;            // fallback digit histograms: 16 rows x 512 words
// LDS words shared by the phases: the sample histograms (16 x kHStride); the
// candidate keys (private [16][kPrivSlots][64] then overflow [16][kOvfCap], u32)
// and positions (the same two arrays in u16); the fallback's digit
// histograms (16 x kFbStride).
constexpr int kPoolWords = kKeyWords + kKeyWords / 2;
static_assert(16 * kHStride <= kPoolWords && 16 * kFbStride <= kPoolWords, "LDS pool too small");
constexpr size_t kPoolBytes = (size_t)kPoolWords * 4;
// The kernel's static arrays take about 19 KiB beside the pool; a block may
// use 160 KiB of LDS.
static_assert(kPoolBytes + 20 * 1024 <= 160 * 1024, "select LDS budget exceeded");
constexpr size_t kSinkBytes = 64 * 8;     // per 16-row group: the mask-word store slots of non-writing lanes
// A candidate's key index is kept in 16 bits (and the 16-bit sample counts
// hold at most 16 * ceil(T/64) keys per row).
constexpr int kMaxSelectT = 65536;

enum RowMode : int { kNone = 0, kTrivial = 1, kActive = 2, kFailed = 3 };

// s_waitcnt immediate (gfx9 encoding): vmcnt(0), expcnt and lgkmcnt not waited.
constexpr int kWaitVmcnt0 = (0x7 << 4) | (0xf << 8);

__device__ __forceinline__ int bin_of(float s, float inv_w) {
  return (int)fmaxf(0.f, fminf(s * inv_w, (float)(kNB - 1)));
}
__device__ __forceinline__ void hist_add(uint32_t* row, int bin) {
  atomicAdd(&row[bin >> 1], 1u << (16 * (bin & 1)));
}
__device__ __forceinline__ int hist_count(const uint32_t* row, int bin) {
  return (int)((row[bin >> 1] >> (16 * (bin & 1))) & 0xffffu);
}

// Causal-prefix chunk of row `row` for 16-key tile `tile`: keys <= row set.
__device__ __forceinline__ uint16_t prefix_chunk(int row, int tile) {
  const int n = row - 16 * tile + 1;    // keys of this tile at or before the row
  return n >= 16 ? (uint16_t)0xffffu : (n <= 0 ? (uint16_t)0 : (uint16_t)((1u << n) - 1u));
}

// OR over the four lanes l, l^16, l^32, l^48 (one query row's four key
// quarters): permlane swaps of the value with itself leave the value and its
// partner in the two results.
__device__ __forceinline__ uint32_t or_row4(uint32_t x) {
  auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  x = r[0] | r[1];
  r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return r[0] | r[1];
}
__device__ __forceinline__ int wave_min(int v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v = min(v, __shfl_xor(v, o, 64));
  return v;
}
__device__ __forceinline__ int wave_max(int v) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) v = max(v, __shfl_xor(v, o, 64));
  return v;
}
// Inclusive suffix sum over the lanes: lane l gets sum_{l' >= l} v_l'.
__device__ __forceinline__ int wave_suffix(int v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_down(v, o, 64);
    if (lane + o < 64) v += y;
  }
  return v;
}
// The lanes of one wave exchange counts through LDS in the resolve, without
// a workgroup barrier.  Without a fence the compiler may treat another lane's
// LDS write as invisible and forward a lane's own earlier store to its load
// (it did: lanes that added nothing read back the zeros they had written).
// This makes every lane's LDS writes before it visible to every lane's reads
// after it.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Inclusive prefix sum over the lanes.
__device__ __forceinline__ int wave_prefix(int v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(v, o, 64);
    if (lane >= o) v += y;
  }
  return v;
}

// Selection parameters of one launch.  The kernel runs in one of three phases:
//   0  fused: every row takes k = k_eff (the reference selector);
//   1  variance-adaptive k, first launch: the sample histograms -> hist and a
//      shift per row (the sample mean), then one pass over every causal score
//      -> each row's population variance -> row_var;
//   2  variance-adaptive k, second launch: row t takes k = k_rows[b*T+t]; the
//      sample histograms come back from hist, then band, main pass, resolve
//      and fallback as in phase 0.
// k_rows is written between the two launches by adaptive_k_kernel, which
// needs every row's variance (its mean over all rows is global).
struct SelArgs {
  int k_eff;              // phase 0
  const int* k_rows;      // phase 2: [B*T]
  float* row_var;         // phase 1: [B*T]
  uint32_t* hist;         // phases 1, 2: 16 * kHStride words per block
  int force_fallback;     // phases 0, 2: every active row takes the fallback (a test hook)
};

template <typename T, int kPhase>
__global__ __launch_bounds__(kGroupThreads) void indexer_select_kernel(IdxArgs p, SelArgs sa, uint32_t* bits,
                                                                     int64_t b_sb, int64_t b_st, uint8_t* ws) {
  // histograms | candidate lists | fallback histograms: kPoolWords words of
  // dynamic LDS (more than the 64 KiB a block gets by default, so the launch
  // raises the block's limit first)
  extern __shared__ uint32_t pool[];
  __shared__ uint32_t sh_rh[kGroupWaves][256];    // resolve: one digit histogram per wave
  __shared__ int st_mode[16], st_k[16], st_need[16], st_ties[16];
  __shared__ float st_lo[16], st_hi[16], st_invw[16];
  __shared__ int st_sure[16 * kGroupWaves];
  __shared__ uint32_t st_cnt[16];                  // overflow-list counters
  __shared__ uint8_t st_pcnt[16][64];              // private-list lengths [row][writer]
  __shared__ uint32_t st_key[16], st_idx[16];
  __shared__ int st_any[3];                       // any active row, any failed row, any index pass

  // (the wave index is read as a scalar so that tile indices, and the
  // branches on them, are known to be uniform across the wave)
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int g = lane >> 4, lr = lane & 15;
  const int ngroups = (p.T + 15) >> 4;
  const int b = blockIdx.x % p.B;
  const int rg_idx = ngroups - 1 - blockIdx.x / p.B;
  const int r0 = rg_idx * 16;
  const int row = r0 + lr;                        // the lane's query row
  uint32_t* bbase = bits + b * b_sb;
  uint16_t* b16 = reinterpret_cast<uint16_t*>(bbase);
  const int64_t row16 = 2 * b_st;                 // uint16 chunks per row
  const int ntl = rg_idx + 1;                     // causal 16-key tiles 0 .. rg_idx
  uint32_t* pkey = pool;                          // private keys [16][kPrivSlots][64]
  uint32_t* okey = pool + kPrivWords;             // overflow keys [16][kOvfCap]
  uint16_t* ppos = reinterpret_cast<uint16_t*>(pool + kKeyWords);     // positions, same layout
  uint16_t* opos = ppos + kPrivWords;
  // where a lane's mask word goes: its row's word, or a sink slot
  uint2* sink = reinterpret_cast<uint2*>(ws + (int64_t)blockIdx.x * kSinkBytes) + lane;

  if (tid < 16) {
    const int r = r0 + tid;
    int k = sa.k_eff;
    if constexpr (kPhase == 2) k = r < p.T ? sa.k_rows[(int64_t)b * p.T + r] : 1;
    // phase 1 scores every row (each row's variance enters the global mean)
    st_mode[tid] = r >= p.T ? kNone : ((kPhase == 1 || r + 1 > k) ? kActive : kTrivial);
    st_k[tid] = k;
    st_cnt[tid] = 0u;
  }
  if (tid < 3) st_any[tid] = 0;
  __syncthreads();
  if (tid < 16 && st_mode[tid] == kActive) st_any[0] = 1;

  // Every chunk after the diagonal tile is zero; trivial rows get their
  // causal prefix now.  (The zeroing is largest for the lightest groups.)
  // Phase 1 writes no mask.
  const int zend = (rg_idx | 3) + 1;              // chunks up to the end of the 64-key word
  if (kPhase != 1 && r0 + wave < p.T) {          // wave w writes row r0 + w
    const int r = r0 + wave;
    const bool triv = st_mode[wave] == kTrivial;
    uint16_t* c16 = b16 + (int64_t)r * row16;
    for (int tile = (triv ? 0 : ntl) + lane; tile < zend; tile += 64)
      c16[tile] = tile >= ntl ? (uint16_t)0 : prefix_chunk(r, tile);
    const int W = 2 * ((p.T + 63) >> 6);
    uint2* c64 = reinterpret_cast<uint2*>(bbase + (int64_t)r * b_st);
    for (int pr = (zend >> 2) + lane; pr < (W >> 1); pr += 64) c64[pr] = uint2{0u, 0u};
  }
  __syncthreads();
  if (!st_any[0]) return;

  RowGroup<T> rgp;
  rgp.init(p, b, r0, lane);
  const bool act = st_mode[lr] == kActive;
  const float inv_w = (float)kNB / ((((rgp.a[0] + rgp.a[1]) + rgp.a[2]) + rgp.a[3]) * 1.0009765625f + 1e-30f);
  if (wave == 0 && g == 0) st_invw[lr] = inv_w;
  uint32_t* hrow = pool + lr * kHStride;
  typedef typename Mfma<T>::Op Op;
  constexpr int kS = Mfma<T>::kSteps;

  // Scores of the lane's row against keys 16t + 4g + e of the tiles t =
  // first, next(first), ... below ntl: f(t, s[4]) per tile.  Two key buffers
  // alternate without copies (the loop handles two tiles per turn): the next
  // tile's keys are requested before this tile's are awaited, always
  // (clamped to the last tile), so that the wait is a fixed count that leaves
  // the new request in flight.
  auto tile = [&](const Op (&kb)[kS], float (&sc)[4]) {
    floatx4 acc[kHi];
    rgp.mma(kb, acc);
    rgp.score4(acc, sc);
  };
  auto sweep = [&](int first, auto&& next, auto&& f) {
    Op ka[kS], kb[kS];
    int t = first;
    rgp.load_keys(16 * min(t, ntl - 1), p.T, lane, ka);
    while (t < ntl) {
      float sc[4];
      const int t1 = next(t);
      rgp.load_keys(16 * min(t1, ntl - 1), p.T, lane, kb);
      tile(ka, sc);
      f(t, sc);
      if (t1 >= ntl) break;
      const int t2 = next(t1);
      rgp.load_keys(16 * min(t2, ntl - 1), p.T, lane, ka);
      tile(kb, sc);
      f(t1, sc);
      t = t2;
    }
  };
  auto round_robin = [](int t) { return t + kGroupWaves; };

  // ---- sample histograms -------------------------------------------------------
  if constexpr (kPhase == 2) {
    // phase 1's histograms (same grid, so the same block index)
    const uint32_t* hsrc = sa.hist + (int64_t)blockIdx.x * (16 * kHStride);
    for (int i = tid; i < 16 * kHStride; i += kGroupThreads) pool[i] = hsrc[i];
  } else {
    for (int i = tid; i < 16 * kHStride; i += kGroupThreads) pool[i] = 0u;
    __syncthreads();
    // (Rows that are not active count into their own, unused histograms.)
    sweep(4 * wave, [](int t) { return t + 4 * kGroupWaves; }, [&](int t, const float (&sc)[4]) {
      if (t != ntl - 1) {
#pragma unroll
        for (int e = 0; e < 4; ++e) hist_add(hrow, bin_of(sc[e], inv_w));
      } else {                                    // the diagonal tile: keys up to the row
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (4 * g + e <= lr) hist_add(hrow, bin_of(sc[e], inv_w));
      }
    });
  }
  __syncthreads();

  if constexpr (kPhase == 1) {
    // ---- row variance (population, over the row's causal scores) --------------
    // Sums of d = s - c and d^2 with c = the sample's mean from its histogram's
    // bin centres (|mean - c| is about a bin width), so that S2/n - (S1/n)^2
    // keeps its precision.  Then the histograms are saved for phase 2.
    __shared__ float st_c[16];
    __shared__ float2 st_part[16 * kGroupWaves];
    if (tid < 256) {
      const int rl = tid >> 4, part = tid & 15;   // 16 threads per row, 64 bins each
      float m = 0.f, n = 0.f;
      for (int bin = part * (kNB / 16); bin < (part + 1) * (kNB / 16); ++bin) {
        const float c = (float)hist_count(&pool[rl * kHStride], bin);
        m = __builtin_fmaf(c, (float)bin + 0.5f, m);
        n += c;
      }
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) {
        m += __shfl_xor(m, o, 64);
        n += __shfl_xor(n, o, 64);
      }
      if (part == 0) st_c[rl] = n > 0.f ? m / (n * st_invw[rl]) : 0.f;
    }
    __syncthreads();
    const float c = st_c[lr];
    float s1 = 0.f, s2 = 0.f;
    // (every row below T is active in this phase; the others are not stored)
    sweep(wave, round_robin, [&](int t, const float (&sc)[4]) {
      const bool diag = t == ntl - 1;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float d = (!diag || 4 * g + e <= lr) ? sc[e] - c : 0.f;
        s1 += d;
        s2 = __builtin_fmaf(d, d, s2);
      }
    });
    s1 += __shfl_xor(s1, 16, 64);
    s2 += __shfl_xor(s2, 16, 64);
    s1 += __shfl_xor(s1, 32, 64);
    s2 += __shfl_xor(s2, 32, 64);
    if (g == 0) st_part[lr * kGroupWaves + wave] = make_float2(s1, s2);
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
    for (int i = tid; i < 16 * kHStride; i += kGroupThreads) hdst[i] = pool[i];
    return;
  }

  // ---- band: wave w takes row w ------------------------------------------------
  {
    const int rl = wave;
    if (st_mode[rl] == kActive) {
      const uint32_t* hr = pool + rl * kHStride;
      int cnt[16];
      int v = 0;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        cnt[i] = hist_count(hr, 16 * lane + i);
        v += cnt[i];
      }
      const int suf = wave_suffix(v, lane);          // samples in bins >= 16 * lane
      const int n_s = __shfl(suf, 0, 64);
      const float n = (float)(r0 + rl + 1), kf = (float)st_k[rl];
      const float pk = kf / n;
      const float rstar = kf * (float)n_s / n;
      const float var = (float)n_s * pk * (1.f - pk) * (1.f - (float)n_s / n);
      const float delta = kBandZ * __builtin_sqrtf(fmaxf(var, 0.f)) + 2.f;
      const float r_hi = rstar - delta, r_lo = rstar + delta;
      // C(b) = samples in bins >= b.  hi: the lowest bin with C(b) <= r_hi;
      // lo: the highest bin with C(b) >= r_lo.
      int bhi = kNB, blo = -1, c = suf;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int bin = 16 * lane + i;
        if ((float)c <= r_hi) bhi = min(bhi, bin);
        if ((float)c >= r_lo) blo = bin;
        c -= cnt[i];
      }
      bhi = wave_min(bhi);
      blo = wave_max(blo);
      if (lane == 0) {
        const float iw = st_invw[rl];
        st_hi[rl] = bhi >= kNB ? __builtin_inff() : (float)bhi / iw;
        st_lo[rl] = blo <= 0 ? -__builtin_inff() : (float)blo / iw;
      }
    }
  }
  __syncthreads();   // the histograms are dead from here: the pool holds the candidate lists

  // ---- main pass: sure winners -> mask words, band -> candidate lists ---------
  // A candidate is kept as the bits of its score (scores are sums of
  // products of sigmoids: never negative, and candidates are never NaN, so
  // the bits order as the values do once -0 is folded into +0) and its key
  // index.  The lane is writer (wave + 16g + lr) mod 64 of its row: the 64
  // lanes of one wave then store to 64 different banks.
  {
    const float lo = act ? st_lo[lr] : __builtin_nanf("");   // NaN: never a candidate
    const float hi = act ? st_hi[lr] : __builtin_inff();
    uint2* wdst = (g == 0 && act) ? reinterpret_cast<uint2*>(bbase + (int64_t)row * b_st) : nullptr;
    const int writer = (wave + 16 * g + lr) & 63;
    uint32_t* pk = pkey + lr * (kPrivSlots * 64) + writer;  // slot i at pk[64 * i]
    uint16_t* pp = ppos + lr * (kPrivSlots * 64) + writer;
    int pc = 0;                                   // candidates of this writer, spilled ones included
    int nsure = 0;
    // One tile's scores -> sure bits in w2, candidates into the lists.  The
    // short form serves tiles below the diagonal while every writer of the
    // wave has room for four more.
    auto classify = [&](int t, int u, const float (&sc)[4], uint32_t (&w2)[2]) {
      const int col0 = 16 * t + 4 * g;
      const bool diag = t == ntl - 1;
      if (!diag && __builtin_amdgcn_ballot_w64(pc > kPrivCap - 4) == 0) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float s = sc[e];
          const bool le = s <= hi;
          w2[u >> 1] |= le ? 0u : (1u << (16 * (u & 1) + 4 * g + e));   // NaN ranks above every number
          // every slot is stored, a non-candidate into the trash slot: no branch
          const bool cand = le && s >= lo;
          const int slot = cand ? pc : kPrivCap;
          pk[64 * slot] = __float_as_uint(s);
          pp[64 * slot] = (uint16_t)(col0 + e);
          pc += cand ? 1 : 0;
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float s = sc[e];
          const bool valid = !diag || 4 * g + e <= lr;
          const bool le = s <= hi;
          w2[u >> 1] |= (valid && !le) ? (1u << (16 * (u & 1) + 4 * g + e)) : 0u;
          if (valid && le && s >= lo) {
            if (pc < kPrivCap) {
              pk[64 * pc] = __float_as_uint(s);
              pp[64 * pc] = (uint16_t)(col0 + e);
            } else {
              const uint32_t at = atomicAdd(&st_cnt[lr], 1u);
              if (at < (uint32_t)kOvfCap) {
                okey[lr * kOvfCap + at] = __float_as_uint(s);
                opos[lr * kOvfCap + at] = (uint16_t)(col0 + e);
              }
            }
            ++pc;
          }
        }
      }
    };
    auto put_word = [&](int qd, const uint32_t (&w2)[2]) {
      const uint32_t lo32 = or_row4(w2[0]), hi32 = or_row4(w2[1]);
      uint2* dst = wdst ? wdst + qd : sink;
      *dst = uint2{lo32, hi32};
      nsure += __popc(lo32) + __popc(hi32);
    };
    // Quads of this wave (wave, wave + 16, ...) that lie below the diagonal
    // tile: even tiles of a quad use key buffer A, odd ones B.  Every turn
    // issues the same memory operations -- four key-tile loads and one word
    // store -- and the loop is entered after one load and one (sink)
    // store, so the compiler's wait for a buffer always leaves the other
    // buffer's load in flight.
    const int nfull = (ntl - 1) >> 2;
    Op kA[kS], kB[kS];
    rgp.load_keys(16 * min(4 * wave, ntl - 1), p.T, lane, kA);
    *sink = uint2{0u, 0u};
    for (int qd = wave; qd < nfull; qd += kGroupWaves) {
      uint32_t w2[2] = {0u, 0u};
      const int t0 = 4 * qd;
      float sc[4];
      rgp.load_keys(16 * (t0 + 1), p.T, lane, kB);
      tile(kA, sc);
      classify(t0, 0, sc, w2);
      rgp.load_keys(16 * (t0 + 2), p.T, lane, kA);
      tile(kB, sc);
      classify(t0 + 1, 1, sc, w2);
      rgp.load_keys(16 * (t0 + 3), p.T, lane, kB);
      tile(kA, sc);
      classify(t0 + 2, 2, sc, w2);
      rgp.load_keys(16 * min(t0 + 4 * kGroupWaves, ntl - 1), p.T, lane, kA);
      tile(kB, sc);
      classify(t0 + 3, 3, sc, w2);
      put_word(qd, w2);
    }
    // The last quad (1-4 tiles, the diagonal tile among them) belongs to
    // wave nfull % 16.
    if (wave == nfull % kGroupWaves) {
      uint32_t w2[2] = {0u, 0u};
      for (int u = 0; u < ntl - 4 * nfull; ++u) {
        const int t = 4 * nfull + u;
        Op kb[kS];
        rgp.load_keys(16 * t, p.T, lane, kb);
        float sc[4];
        tile(kb, sc);
        classify(t, u, sc, w2);
      }
      put_word(nfull, w2);
    }
    if (g == 0) st_sure[lr * kGroupWaves + wave] = act ? nsure : 0;
    st_pcnt[lr][writer] = (uint8_t)min(pc, kPrivCap);
  }
  // The resolve ORs winners into the words stored above, by atomics that
  // execute in L2, from other waves.  A workgroup-scope barrier does not wait
  // for this wave's stores to reach L2 (they are visible to the workgroup
  // through the CU's cache first), so a late store could overwrite the ORed
  // bits: wait for them explicitly before the barrier.
  __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
  __syncthreads();

  // ---- resolve: wave w takes row w -----------------------------------------------
  {
    const int rl = wave;
    if (st_mode[rl] == kActive) {
      int n_sure = 0;
#pragma unroll
      for (int w = 0; w < kGroupWaves; ++w) n_sure += st_sure[rl * kGroupWaves + w];
      // lane j reads writer j's private list, and every 64th overflow slot
      const int np = st_pcnt[rl][lane];
      const int n_ovf = (int)st_cnt[rl];
      int n_all = np;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) n_all += __shfl_xor(n_all, o, 64);
      n_all += n_ovf;
      int need = st_k[rl] - n_sure;
      if (sa.force_fallback || n_ovf > kOvfCap || need < 0 || n_all < need) {
        if (lane == 0) { st_mode[rl] = kFailed; st_any[1] = 1; }
      } else if (need > 0) {
        const uint32_t* rk = pkey + rl * (kPrivSlots * 64) + lane;
        const uint16_t* rp = ppos + rl * (kPrivSlots * 64) + lane;
        const uint32_t* xk = okey + rl * kOvfCap;
        const uint16_t* xp = opos + rl * kOvfCap;
        // The lane's private list -- writer `lane`'s, np <= kPrivCap entries --
        // is read from LDS once into registers (keys in ck, two 16-bit indices
        // per cp word); the overflow slots lane, lane + 64, ... stay in LDS.
        uint32_t ck[kPrivCap], cp[kPrivCap / 2];
#pragma unroll
        for (int i = 0; i < kPrivCap; ++i) ck[i] = rk[64 * i] & 0x7fffffffu;
#pragma unroll
        for (int i = 0; i < kPrivCap / 2; ++i) cp[i] = (uint32_t)rp[128 * i] | ((uint32_t)rp[128 * i + 64] << 16);
        // f(key, index) for each of the row's candidates held by this lane
        auto each = [&](auto&& f) {
#pragma unroll
          for (int i = 0; i < kPrivCap; ++i)
            if (i < np) f(ck[i], (int)((cp[i >> 1] >> (16 * (i & 1))) & 0xffffu));
          for (int i = lane; i < n_ovf; i += 64) f(xk[i] & 0x7fffffffu, (int)xp[i]);
        };
        // theta = the need-th largest candidate key.  Radix select MSB-first on
        // key - kmin over the bits of the candidates' key range kmax - kmin,
        // 8-bit digits counted in LDS: the first digit splits the actual range
        // of the candidates into 256 bins of about equal width.  A digit whose
        // keys are all still needed ends the search: theta is then its least key
        // and every key equal to it is taken.
        uint32_t kmin = ~0u, kmax = 0u;
        each([&](uint32_t kk, int) { kmin = min(kmin, kk); kmax = max(kmax, kk); });
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          kmin = min(kmin, (uint32_t)__shfl_xor((int)kmin, o, 64));
          kmax = max(kmax, (uint32_t)__shfl_xor((int)kmax, o, 64));
        }
        auto each_rel = [&](auto&& f) { each([&](uint32_t kk, int ix) { f(kk - kmin, ix); }); };
        const uint32_t range = kmax - kmin;
        int rem = range ? 32 - __builtin_clz(range) : 0;     // low bits still open
        uint32_t prefix = 0u;
        bool all_ties = false;
        uint32_t* rh = sh_rh[wave];
        while (rem > 0) {
          const int nb = rem < 8 ? rem : 8, shift = rem - nb;
          const uint32_t hmask = rem >= 32 ? 0u : ~0u << rem;
#pragma unroll
          for (int i = 0; i < 4; ++i) rh[4 * lane + i] = 0u;
          wave_lds_sync();
          each_rel([&](uint32_t kk, int) {
            if ((kk & hmask) == prefix) atomicAdd(&rh[(kk >> shift) & ((1u << nb) - 1u)], 1u);
          });
          wave_lds_sync();
          int cb[4], vsum = 0;
#pragma unroll
          for (int i = 0; i < 4; ++i) { cb[i] = (int)rh[4 * lane + i]; vsum += cb[i]; }
          const int suf = wave_suffix(vsum, lane);            // keys in digits >= 4 * lane
          // the highest digit d with count(digits >= d) >= need
          int dsel = -1, above = 0, cnt = 0, c = suf;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            if (c >= need) { dsel = 4 * lane + i; above = c - cb[i]; cnt = cb[i]; }
            c -= cb[i];
          }
          const int d = wave_max(dsel);
          need -= __shfl(above, d >> 2, 64);
          const int cnt_d = __shfl(cnt, d >> 2, 64);
          prefix |= (uint32_t)d << shift;
          rem = shift;
          if (rem > 0 && cnt_d == need) {
            const uint32_t fixed = ~0u << rem;
            uint32_t least = ~0u;
            each_rel([&](uint32_t kk, int) { if ((kk & fixed) == prefix) least = min(least, kk); });
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) least = min(least, (uint32_t)__shfl_xor((int)least, o, 64));
            prefix = least;
            all_ties = true;
            break;
          }
        }
        const uint32_t theta = prefix + kmin;
        int ties = 0;
        if (!all_ties) {
          each([&](uint32_t kk, int) { ties += kk == theta ? 1 : 0; });
#pragma unroll
          for (int o = 1; o < 64; o <<= 1) ties += __shfl_xor(ties, o, 64);
        }
        uint32_t istar = 0xffffffffu;
        if (ties > need) {       // rare: the need lowest indices among the ties, 9-bit digits
          uint32_t ip = 0u;
          for (int lvl = 0; lvl < 2; ++lvl) {
            const int shift = 9 * (1 - lvl);
#pragma unroll
            for (int i = 0; i < 4; ++i) rh[4 * lane + i] = 0u;   // 512 digits as 16-bit counts
            wave_lds_sync();
            each([&](uint32_t kk, int ix) {
              if (kk == theta && (lvl == 0 || ((uint32_t)ix >> 9) == ip)) {
                const int dg = (ix >> shift) & 511;
                atomicAdd(&rh[dg >> 1], 1u << (16 * (dg & 1)));
              }
            });
            wave_lds_sync();
            int cb[8], vsum = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              const int dg = 8 * lane + i;
              cb[i] = (int)((rh[dg >> 1] >> (16 * (dg & 1))) & 0xffffu);
              vsum += cb[i];
            }
            // the lowest digit d with count(digits <= d) >= need
            int dsel = 512, below = 0, c = wave_prefix(vsum, lane) - vsum;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              if (c + cb[i] >= need && dsel == 512) { dsel = 8 * lane + i; below = c; }
              c += cb[i];
            }
            const int d = wave_min(dsel);
            need -= __shfl(below, d >> 3, 64);
            ip = (ip << 9) | (uint32_t)d;
          }
          istar = ip;
        }
        // Winners -> the row's stored mask words.  They are ORed into a
        // bitmap in this row's private-key region of LDS (kBitmapWords words,
        // free: the lists are in ck/cp now), then each nonzero word of the
        // bitmap is ORed into the stored word by one read-modify-write: one
        // wave owns the row here, and the main pass's stores, made by this
        // workgroup and complete before the barrier (vmcnt(0)), are visible
        // to its loads after it.  Longer rows take several chunks.  (Global
        // atomics per winner instead: c3 0.333 ms, B=4 T=8192 0.371 ms.)
        constexpr int kBitmapWords = kPrivSlots * 64;
        uint32_t* brow = bbase + (int64_t)(r0 + rl) * b_st;
        uint32_t* bm = pkey + rl * kBitmapWords;
        const int nw = ((r0 + rl) >> 5) + 1;            // words that can hold a causal key
        for (int c0 = 0; c0 < nw; c0 += kBitmapWords) {
          const int cw = min(kBitmapWords, nw - c0);
          for (int j = lane; j < cw; j += 64) bm[j] = 0u;
          wave_lds_sync();
          each([&](uint32_t kk, int ix) {
            const int wi = (ix >> 5) - c0;
            if ((kk > theta || (kk == theta && (uint32_t)ix <= istar)) && (uint32_t)wi < (uint32_t)cw)
              atomicOr(&bm[wi], 1u << (ix & 31));
          });
          wave_lds_sync();
          for (int j = lane; j < cw; j += 64) {
            const uint32_t v = bm[j];
            if (v) {
              uint32_t* pw = brow + c0 + j;
              *pw = __hip_atomic_load(pw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) | v;
            }
          }
          wave_lds_sync();                               // the bitmap's reads before the next chunk's zeros
        }
      }
    }
  }
  __syncthreads();
  if (!st_any[1]) return;

  // ---- fallback: exact radix select over recomputed scores of failed rows ------
  const bool fb = st_mode[lr] == kFailed;
  if (tid < 16) {
    st_need[tid] = st_k[tid];
    st_key[tid] = 0u;
    st_idx[tid] = 0u;
  }
  for (int level = 0; level < 4; ++level) {
    for (int i = tid; i < 16 * kFbStride; i += kGroupThreads) pool[i] = 0u;
    __syncthreads();
    const uint32_t pre = st_key[lr];
    const int ls = 24 - 8 * level;
    sweep(wave, round_robin, [&](int t, const float (&sc)[4]) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (fb && 16 * t + 4 * g + e <= row) {
          const uint32_t kk = score_key(sc[e]);
          if (level == 0 || (kk >> (ls + 8)) == pre) atomicAdd(&pool[lr * kFbStride + ((kk >> ls) & 255u)], 1u);
        }
      }
    });
    __syncthreads();
    if (tid < 16 && st_mode[tid] == kFailed) {
      int cum = 0, d = 0, nd = st_need[tid];
      for (int bin = 255; bin >= 0; --bin) {
        const int c = (int)pool[tid * kFbStride + bin];
        if (cum + c >= nd) { d = bin; st_ties[tid] = c; break; }
        cum += c;
      }
      st_need[tid] = nd - cum;
      st_key[tid] = (st_key[tid] << 8) | (uint32_t)d;
      if (level == 3 && st_ties[tid] > st_need[tid]) st_any[2] = 1;
    }
    __syncthreads();
  }
  // ties at the threshold beyond the need: the need lowest indices (< 2^16)
  const bool ix_row = fb && st_ties[lr] > st_need[lr];
  if (st_any[2]) {
    for (int lvl = 0; lvl < 2; ++lvl) {
      for (int i = tid; i < 16 * kFbStride; i += kGroupThreads) pool[i] = 0u;
      __syncthreads();
      const uint32_t theta = st_key[lr], ip = st_idx[lr];
      const int shift = 9 * (1 - lvl);
      sweep(wave, round_robin, [&](int t, const float (&sc)[4]) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int col = 16 * t + 4 * g + e;
          if (ix_row && col <= row && score_key(sc[e]) == theta && (lvl == 0 || ((uint32_t)col >> 9) == ip))
            atomicAdd(&pool[lr * kFbStride + ((col >> shift) & 511)], 1u);
        }
      });
      __syncthreads();
      if (tid < 16 && st_mode[tid] == kFailed && st_ties[tid] > st_need[tid]) {
        int cum = 0, d = 0;
        const int nd = st_need[tid];
        for (int bin = 0; bin < 512; ++bin) {
          const int c = (int)pool[tid * kFbStride + bin];
          if (cum + c >= nd) { d = bin; break; }
          cum += c;
        }
        st_idx[tid] = (st_idx[tid] << 9) | (uint32_t)d;
        if (lvl == 0) st_need[tid] = nd - cum;      // the first digit's lower ties are all taken
      }
      __syncthreads();
    }
  }
  // marking: every word of a failed row is rewritten
  {
    const uint32_t theta = st_key[lr];
    const uint32_t istar = ix_row ? st_idx[lr] : 0xffffffffu;
    uint2* wdst = (g == 0 && fb) ? reinterpret_cast<uint2*>(bbase + (int64_t)row * b_st) : nullptr;
    for (int qd = wave; 4 * qd < ntl; qd += kGroupWaves) {
      uint32_t w2[2] = {0u, 0u};
      for (int u = 0; u < 4; ++u) {
        const int t = 4 * qd + u;
        if (t >= ntl) break;
        Op kb[kS];
        rgp.load_keys(16 * t, p.T, lane, kb);
        floatx4 acc[kHi];
        rgp.mma(kb, acc);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int col = 16 * t + 4 * g + e;
          const uint32_t kk = score_key(rgp.score(acc, e));
          const bool sel = fb && col <= row && (kk > theta || (kk == theta && (uint32_t)col <= istar));
          w2[u >> 1] |= sel ? (1u << (16 * (u & 1) + 4 * g + e)) : 0u;
        }
      }
      const uint32_t lo32 = or_row4(w2[0]), hi32 = or_row4(w2[1]);
      uint2* dst = wdst ? wdst + qd : sink;
      *dst = uint2{lo32, hi32};
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
// Device memory of gsa_indexer_select_noalloc: the selector's sink slots
// (kSinkBytes per 16-row group) for callers that cannot allocate.  Every
// device that loads the library holds one copy, at its own address, until
// the process ends.  Host code never passes `scratch` itself to a kernel
// (in host code it names a host-side stand-in): it takes each device's
// address from hipGetSymbolAddress once and passes that.
// ---------------------------------------------------------------------------
constexpr size_t kNoAllocScratchBytes = (size_t)4 << 20;   // B * ceil(T/16) <= 8192 groups
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

// ---------------------------------------------------------------------------
// Host entry points
// ---------------------------------------------------------------------------
#include <atomic>
#include <mutex>

using namespace gsa_host;

// Process-wide test hook: every active row of the fused selector takes the
// exact fallback path (gsa_debug_force_select_fallback).
static std::atomic<int> g_force_fallback{0};

static int check_indexer_args(const void* q, int64_t q_sb, int64_t q_st, const void* k, int64_t k_sb,
                              int64_t k_st, const void* w, const float* bias, int B, int T, int Hi,
                              int di, int dtype) {
  if (!q || !k || !w || !bias) return GSA_ERR_NULL;
  if (dtype_size(dtype) == 0) return GSA_ERR_DTYPE;
  if (B < 1 || T < 1 || Hi != gsa::kHi || di != gsa::kDi) return GSA_ERR_SHAPE;
  if (!vec_ok(q, q_sb, q_st, dtype) || !vec_ok(k, k_sb, k_st, dtype)) return GSA_ERR_ALIGN;
  if (!aligned(w, dtype_size(dtype)) || !aligned(bias, 4)) return GSA_ERR_ALIGN;
  if (k_st < 0 || k_st * dtype_size(dtype) * 16 >= (int64_t)1 << 31) return GSA_ERR_SHAPE;   // 32-bit tile offsets
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
  const int vec = aligned(scores, 16) && (s_st % 4) == 0 && (s_sb % 4) == 0;
  dim3 grid((waves + 3) / 4), block(256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == GSA_DTYPE_BF16)
    hipLaunchKernelGGL(gsa::indexer_scores_kernel<uint16_t>, grid, block, 0, s, a, causal, scores, s_sb, s_st, vec);
  else
    hipLaunchKernelGGL(gsa::indexer_scores_kernel<float>, grid, block, 0, s, a, causal, scores, s_sb, s_st, vec);
  return launch_status();
}

// The selector's blocks use more LDS than the 64 KiB default: raise each
// instantiation's limit once per device.  (A benign race: concurrent first
// calls both set the same attribute.)
static constexpr int kMaxDevices = 64;

template <typename Kern>
static int raise_lds_limit(Kern kern, bool (&done)[kMaxDevices]) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return GSA_ERR_SHAPE;
  if (!done[dev]) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)gsa::kPoolBytes);
    if (e != hipSuccess) return -static_cast<int>(e);
    done[dev] = true;
  }
  return GSA_OK;
}

// One launch of the fused selector in phase kPhase.
template <typename T, int kPhase>
static int launch_select_t(const gsa::IdxArgs& a, const gsa::SelArgs& sa, uint32_t* bits, int64_t b_sb,
                           int64_t b_st, uint8_t* ws, hipStream_t s) {
  static bool lds_set[kMaxDevices] = {};
  const int st = raise_lds_limit(gsa::indexer_select_kernel<T, kPhase>, lds_set);
  if (st) return st;
  const dim3 grid(a.B * ((a.T + 15) / 16)), block(gsa::kGroupThreads);
  hipLaunchKernelGGL((gsa::indexer_select_kernel<T, kPhase>), grid, block, gsa::kPoolBytes, s, a, sa, bits, b_sb,
                     b_st, ws);
  return launch_status();
}

template <int kPhase>
static int launch_select(const gsa::IdxArgs& a, gsa::SelArgs sa, int dtype, uint32_t* bits, int64_t b_sb,
                         int64_t b_st, uint8_t* ws, hipStream_t s) {
  sa.force_fallback = g_force_fallback.load(std::memory_order_relaxed);
  if (dtype == GSA_DTYPE_BF16) return launch_select_t<uint16_t, kPhase>(a, sa, bits, b_sb, b_st, ws, s);
  return launch_select_t<float, kPhase>(a, sa, bits, b_sb, b_st, ws, s);
}

// The candidate lists live in LDS: the workspace holds only the store slots of
// lanes without a mask word to write (kSinkBytes per 16-row group).
extern "C" size_t gsa_indexer_select_workspace_bytes(int B, int T) {
  if (B < 1 || T < 1) return 0;
  return (size_t)B * (size_t)((T + 15) / 16) * gsa::kSinkBytes;
}

extern "C" int gsa_debug_force_select_fallback(int on) {
  return g_force_fallback.exchange(on ? 1 : 0);
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
                             const int32_t* idx_out, const int32_t* count_out) {
  int st = check_indexer_args(q_idx, q_sb, q_st, k_idx, k_sb, k_st, w, bias, B, T, Hi, di, dtype);
  if (st) return st;
  if (!bits) return GSA_ERR_NULL;
  if ((idx_out == nullptr) != (count_out == nullptr)) return GSA_ERR_NULL;
  if (T > gsa::kMaxSelectT) return GSA_ERR_SHAPE;
  const int W = 2 * ((T + 63) / 64);
  if (b_st < W || (B > 1 && b_sb < (int64_t)T * b_st)) return GSA_ERR_SHAPE;
  if (!aligned(bits, 8) || (b_st % 2) || (b_sb % 2)) return GSA_ERR_ALIGN;
  if (idx_out && (!aligned(idx_out, 4) || !aligned(count_out, 4))) return GSA_ERR_ALIGN;
  if ((int64_t)B * T > 0x7fffffffLL) return GSA_ERR_SHAPE;
  return GSA_OK;
}

// The launches of the fixed-k select, after its arguments are checked; ws
// holds at least gsa_indexer_select_workspace_bytes(B, T) bytes.
static int select_fixed(const gsa::IdxArgs& a, int k_eff, int dtype, uint32_t* bits, int64_t b_sb,
                        int64_t b_st, int32_t* idx_out, int32_t* count_out, uint8_t* ws, hipStream_t s) {
  int st = launch_select<0>(a, gsa::SelArgs{k_eff, nullptr, nullptr, nullptr, 0}, dtype, bits, b_sb, b_st, ws, s);
  if (st || !idx_out) return st;
  const int W = 2 * ((a.T + 63) / 64);
  hipLaunchKernelGGL(gsa::bits_to_indices_kernel, dim3(a.B * a.T), dim3(256), 0, s, bits, b_sb, b_st, a.T, W,
                     k_eff, nullptr, idx_out, count_out);
  return launch_status();
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
                             b_st, idx_out, count_out);
  if (st) return st;
  if (!ws) return GSA_ERR_NULL;
  if (!aligned(ws, 16)) return GSA_ERR_ALIGN;
  if (k_eff < 1 || k_eff > T) return GSA_ERR_K;
  if (ws_bytes < gsa_indexer_select_workspace_bytes(B, T)) return GSA_ERR_SHAPE;
  gsa::IdxArgs a = make_idx_args(q_idx, q_sb, q_st, k_idx, k_sb, k_st, w, w_sb, w_st, bias, scale, B, T);
  return select_fixed(a, k_eff, dtype, bits, b_sb, b_st, idx_out, count_out, static_cast<uint8_t*>(ws),
                      static_cast<hipStream_t>(stream));
}

// Each device's address of `scratch`, looked up on the first call of
// gsa_indexer_select_noalloc with that device current.
static std::mutex g_scratch_mu;
static uint8_t* g_scratch_ptr[kMaxDevices] = {};

static int noalloc_scratch(uint8_t** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return -static_cast<int>(e);
  if (dev < 0 || dev >= kMaxDevices) return GSA_ERR_SHAPE;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return -static_cast<int>(e);
    if (!ptr) return -static_cast<int>(hipErrorInvalidSymbol);
    g_scratch_ptr[dev] = static_cast<uint8_t*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return GSA_OK;
}

extern "C" size_t gsa_indexer_select_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

extern "C" int gsa_indexer_select_noalloc(const void* q_idx, int64_t q_sb, int64_t q_st,
                                          const void* k_idx, int64_t k_sb, int64_t k_st,
                                          const void* w, int64_t w_sb, int64_t w_st,
                                          const float* bias, float scale,
                                          int B, int T, int Hi, int di, int k_eff, int dtype,
                                          uint32_t* bits, int64_t b_sb, int64_t b_st,
                                          int32_t* idx_out, int32_t* count_out, void* stream) {
  int st = check_select_args(q_idx, q_sb, q_st, k_idx, k_sb, k_st, w, bias, B, T, Hi, di, dtype, bits, b_sb,
                             b_st, idx_out, count_out);
  if (st) return st;
  if (k_eff < 1 || k_eff > T) return GSA_ERR_K;
  if (gsa_indexer_select_workspace_bytes(B, T) > kNoAllocScratchBytes) return GSA_ERR_SCRATCH;
  uint8_t* ws = nullptr;
  if ((st = noalloc_scratch(&ws))) return st;
  gsa::IdxArgs a = make_idx_args(q_idx, q_sb, q_st, k_idx, k_sb, k_st, w, w_sb, w_st, bias, scale, B, T);
  return select_fixed(a, k_eff, dtype, bits, b_sb, b_st, idx_out, count_out, ws, static_cast<hipStream_t>(stream));
}

// Adaptive workspace: the fixed selector's, then the sample histograms kept
// between the launches (16 rows x kHStride words per 16-row group), then the
// per-row variances and k values ([B*T] each, used when the caller does not
// take them).
static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

static size_t hist_ws_bytes(int B, int T) {
  return (size_t)B * (size_t)((T + 15) / 16) * 16 * gsa::kHStride * sizeof(uint32_t);
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
                             b_st, idx_out, count_out);
  if (st) return st;
  if (!ws) return GSA_ERR_NULL;
  if (!aligned(ws, 16)) return GSA_ERR_ALIGN;
  if (k_base < 1 || k_min < 1 || k_max < k_min) return GSA_ERR_K;
  if ((k_out && !aligned(k_out, 4)) || (var_out && !aligned(var_out, 4))) return GSA_ERR_ALIGN;
  if (ws_bytes < gsa_indexer_select_adaptive_workspace_bytes(B, T)) return GSA_ERR_SHAPE;
  const int k_cap = k_max < T ? k_max : T;
  gsa::IdxArgs a = make_idx_args(q_idx, q_sb, q_st, k_idx, k_sb, k_st, w, w_sb, w_st, bias, scale, B, T);
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint8_t* base = static_cast<uint8_t*>(ws);
  size_t off = align256(gsa_indexer_select_workspace_bytes(B, T));
  uint32_t* hist = reinterpret_cast<uint32_t*>(base + off);
  off += align256(hist_ws_bytes(B, T));
  float* var = var_out ? var_out : reinterpret_cast<float*>(base + off);
  off += align256((size_t)B * T * sizeof(float));
  int32_t* krow = k_out ? k_out : reinterpret_cast<int32_t*>(base + off);

  if ((st = launch_select<1>(a, gsa::SelArgs{0, nullptr, var, hist, 0}, dtype, bits, b_sb, b_st, base, s)))
    return st;
  if ((st = launch_adaptive_k(var, B * T, k_base, k_min, k_max, k_cap, krow, s))) return st;
  st = launch_select<2>(a, gsa::SelArgs{0, krow, nullptr, hist, 0}, dtype, bits, b_sb, b_st, base, s);
  if (st || !idx_out) return st;
  const int W = 2 * ((T + 63) / 64);
  hipLaunchKernelGGL(gsa::bits_to_indices_kernel, dim3(B * T), dim3(256), 0, s, bits, b_sb, b_st, T, W, k_cap,
                     krow, idx_out, count_out);
  return launch_status();
}
