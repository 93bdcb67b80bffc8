// nie_paged.hip — paged-attention kernels for MI355X (gfx950 / CDNA4).
//
// Kernels
//   kv_append_kernel        slot-mapped scatter of new K/V rows into the cache
//   kv_gather_kernel        logical -> contiguous copy of one sequence
//   kv_copy_blocks_kernel   whole-block copies (export / import of sequences)
//   paged_decode_kernel     split-K decode attention, one workgroup per
//                           (sequence, key split, KV-head group), one wave
//                           per KV head
//   decode_merge_kernel     exact fp32 merge of the split partials
//   varlen_prefill_kernel   chunked-prefill attention over packed varlen rows
//
// Attention math (both attention kernels) runs on the matrix cores with the
// transposed formulation
//     S^T = K . Q^T       (rows = keys,  cols = query rows)
//     O^T = V^T . P^T     (rows = dims,  cols = query rows)
// using v_mfma_f32_16x16x16_bf16 (bf16) or v_mfma_f32_16x16x4_f32 (fp32).
// In this form the C-layout of S^T (lane l holds keys 4*(l/16)+i of query
// row l%16) is exactly the B-layout P^T needs, and the O^T accumulator keeps
// every query row in the lanes with the same l%16, so the online-softmax
// rescale is lane-local and the only cross-lane traffic per 16-key tile is
// a 4-way max.  A query "row" is one (query token, query head) pair of a GQA
// group; a wave owns 16 rows.
//
// The reference's rounding points are kept: the q.k score is rounded to the
// storage dtype, multiplied by the scale and rounded again
// (layers/paged_attention.py:97-98, layers/attention.py:400); softmax is fp32
// (paged_attention.py:109-111); the output is rounded once at the end.

#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <atomic>
#include <initializer_list>
#include <mutex>
#include <vector>
#include <type_traits>

#include "nie_paged.h"

#define NIE_API extern "C" __attribute__((visibility("default")))

namespace {

// ---------------------------------------------------------------------------
// Host-side error reporting
// ---------------------------------------------------------------------------
thread_local char g_last_error[1024] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int launched(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    return fail(NIE_ELAUNCH, "%s launch failed: %s", what, hipGetErrorString(err));
  }
  return NIE_OK;
}

__host__ __device__ inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---------------------------------------------------------------------------
// Device helpers
// ---------------------------------------------------------------------------
typedef short v4s __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;
constexpr int kTileKeys = 16;      // keys per attention tile (one MFMA M/N edge)
constexpr int kLdsPadBytes = 16;   // row padding that makes the V^T reads bank-conflict free
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kNegInf = -__builtin_huge_valf();

struct bf16_t {
  uint16_t bits;
};

template <typename T>
struct Elt;
template <>
struct Elt<float> {
  static constexpr int kBytes = 4;
  static constexpr bool kIsBf16 = false;
};
template <>
struct Elt<bf16_t> {
  static constexpr int kBytes = 2;
  static constexpr bool kIsBf16 = true;
};

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// float -> bf16, round to nearest even (torch's conversion), on gfx950's
// v_cvt_pk_bf16_f32.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float x) {
  return __builtin_bit_cast(uint16_t, (__bf16)x);
}

// Two floats -> two bf16 in one dword (a in the low half).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
}

__device__ __forceinline__ float round_to_bf16(float x) {
  return (float)(__bf16)x;
}

// Rounds x to bf16 (round to nearest even) and returns the rounded value as
// a float in one instruction: v_cvt_pk_bf16_f32 with 0 for the low half
// leaves bf16(x) in the high half, which read as a float is the value itself.
__device__ __forceinline__ float round_bf16_in_f32(float x) {
  return __uint_as_float(pack_bf16x2(0.f, x));
}

typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

// Four floats -> the bf16 MFMA operand (element i = x[i]).
__device__ __forceinline__ v4s pack_bf16x4(float x0, float x1, float x2, float x3) {
  return __builtin_bit_cast(v4s, u32x2_t{pack_bf16x2(x0, x1), pack_bf16x2(x2, x3)});
}

typedef unsigned v4u __attribute__((ext_vector_type(4)));

// Two 4-element bf16 operands (sub-tile a's keys, then sub-tile b's) as one
// 8-element 16x16x32 operand.  With it, K slot 8(l/16) + e of an MFMA is key
// 4(l/16) + e of sub-tile a for e < 4 and key 4(l/16) + e - 4 of sub-tile b
// otherwise, the same on the V^T and the P^T side.
__device__ __forceinline__ bf16x8_t join_bf16x4(v4s a, v4s b) {
  const u32x2_t lo = __builtin_bit_cast(u32x2_t, a);
  const u32x2_t hi = __builtin_bit_cast(u32x2_t, b);
  return __builtin_bit_cast(bf16x8_t, v4u{lo[0], lo[1], hi[0], hi[1]});
}

// 2^x on v_exp_f32 (results below 2^-126 flush to zero, which the softmax
// sums cannot resolve anyway).
__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// e^x to about one ulp, for the probabilities that are rounded to bf16 as
// the reference rounds them (torch's exp is accurate to about an ulp; 2^(x
// log2 e) through fast_exp2 would carry the rounding of x log2 e, an error
// of |x| 2^-24 in the exponent, and move the bf16 rounding of about one
// probability in 10^4).  x log2 e is formed as hi + lo: hi the rounded
// product, lo its rounding error (fma) plus x times the part of log2 e that
// float drops; then e^x = 2^hi (1 + lo ln 2) to within lo^2.  Results below
// 2^-126 flush to zero (no bf16 probability of a sum of at least 1 gets
// there with an effect on the output).
__device__ __forceinline__ float exp_ref(float x) {
  constexpr float kL2eHi = 1.44269502162933349609375f;  // log2(e) rounded to float
  constexpr float kL2eLo = 1.925963033500011079e-8f;    // log2(e) - kL2eHi
  constexpr float kLn2 = 0.693147180559945309f;
  // -inf (a masked key) gives 0 through a finite argument; NaN propagates
  x = __builtin_elementwise_maximum(x, -200.f);
  const float hi = x * kL2eHi;
  const float lo = fmaf(x, kL2eLo, fmaf(x, kL2eHi, -hi));
  const float e = __builtin_amdgcn_exp2f(hi);
  return fmaf(e, lo * kLn2, e);
}

// e / l rounded to nearest, given r = 1 / l rounded to nearest: the product
// e r (two roundings) corrected by one Newton step on its exact residual
// e - q l (fma), as torch's division e / l rounds once.
__device__ __forceinline__ float div_ref(float e, float l, float r) {
  const float q = e * r;
  return fmaf(fmaf(-q, l, e), r, q);
}

// Rounds a value to the storage dtype (identity for fp32).
template <typename T>
__device__ __forceinline__ float round_storage(float x) {
  if constexpr (Elt<T>::kIsBf16) {
    return round_to_bf16(x);
  } else {
    return x;
  }
}

__device__ __forceinline__ int lane_id() { return threadIdx.x & (kWave - 1); }

// Sum / max of a value over the four lane groups with equal l%16
// (lanes l, l^16, l^32, l^48).  v_permlane16_swap / v_permlane32_swap of a
// value with itself give every lane its l^16 (then l^32) partner in one of
// the two results, so the reduction needs no LDS crossbar; the order of the
// operations (pairs first) makes every lane's result identical.
__device__ __forceinline__ float sum_over_groups(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Maximum of two scores.  Scores are never NaN where it matters (masked keys
// are -inf; a NaN input propagates, as through the reference's softmax), so
// the IEEE-754 2019 maximum serves, which gfx950 runs as v_maximum3_f32
// without the operand canonicalization fmaxf needs in IEEE mode.
__device__ __forceinline__ float score_max(float a, float b) { return __builtin_elementwise_maximum(a, b); }

__device__ __forceinline__ float max_over_groups(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = score_max(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return score_max(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// The dispatcher hands workgroup i of a launch to XCD i % kXcds (round robin
// over MI355X's eight XCDs, each with its own L2).  xcd_logical (and
// xcd_logical32, the same in 32-bit arithmetic) maps a 1-D
// workgroup index to a logical index so that each XCD receives one contiguous
// range of [0, n): workgroups that share inputs (the items of one KV head)
// then share an L2.  Only placement depends on it, never correctness.
constexpr int64_t kXcds = 8;

__device__ __forceinline__ uint32_t xcd_logical32(uint32_t i, uint32_t n) {
  constexpr uint32_t kX = (uint32_t)kXcds;
  const uint32_t x = i % kX, j = i / kX;
  const uint32_t q = n / kX, r = n % kX;
  return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + j;
}

__device__ __forceinline__ int64_t xcd_logical(int64_t i, int64_t n) {
  const int64_t x = i % kXcds, j = i / kXcds;
  const int64_t q = n / kXcds, r = n % kXcds;
  return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + j;
}

__device__ __forceinline__ int64_t uniform64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Locates work item `item` in a flattened list where sequence b owns
// per_seq(b) consecutive items.  Every lane of the wave returns the same
// (b, k, first_item_of_b, count_of_b); b == -1 if item is past the end.
template <typename CountFn>
__device__ __forceinline__ void locate_item(int64_t item, int64_t num_seqs, CountFn per_seq,
                                            int64_t* seq, int64_t* local, int64_t* first,
                                            int64_t* count) {
  const int lane = lane_id();
  int64_t base = 0;
  for (int64_t b0 = 0; b0 < num_seqs; b0 += kWave) {
    const int64_t b = b0 + lane;
    const int64_t n = (b < num_seqs) ? per_seq(b) : 0;
    int64_t incl = n;  // inclusive prefix sum over the wave
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int64_t up = __shfl_up(incl, off);
      if (lane >= off) incl += up;
    }
    const int64_t excl = incl - n;
    const int64_t total = __shfl(incl, kWave - 1);
    if (item < base + total) {
      const bool mine = (b < num_seqs) && (item >= base + excl) && (item < base + incl);
      const uint64_t mask = __ballot(mine);
      const int src = __builtin_ctzll(mask);
      // The values are wave-uniform; readfirstlane lets the compiler keep
      // everything derived from them (table lookups, addresses) in SGPRs.
      const int64_t f = base + __shfl(excl, src);
      const int64_t c = __shfl(n, src);
      *seq = (int64_t)__builtin_amdgcn_readfirstlane((int)(b0 + src));
      *first = uniform64(f);
      *count = uniform64(c);
      *local = uniform64(item - f);
      return;
    }
    base += total;
  }
  *seq = -1;
  *local = 0;
  *first = 0;
  *count = 0;
}

// Cache geometry of one layer.  Positions are int32 (a sequence is shorter
// than 2^31 tokens); element offsets are int64 (pools exceed 2^31 elements).
struct CacheGeom {
  int64_t layer_offset;  // elements before this layer: layer * num_blocks * block_size * row_elems
  int64_t row_elems;     // kv_heads * head_dim: elements between consecutive slots
  int32_t num_blocks;
  int32_t block_size;
  int32_t bs_shift;      // log2(block_size) when it is a power of two, else -1
  int32_t kv_heads;
  int32_t row_elems32;   // row_elems as int32 (kv_heads * head_dim < 2^31 / 16)
};

// Element offset of (logical position `pos` of the sequence whose block
// table is `table`[0..table_len), kv head 0, dim 0).  Table index and
// physical block are clamped so a bad table cannot leave the pool.
__device__ __forceinline__ int64_t token_offset(const CacheGeom& g, const int32_t* table,
                                                int table_len, int pos) {
  int lb, off;
  if (g.bs_shift >= 0) {
    lb = pos >> g.bs_shift;
    off = pos & (g.block_size - 1);
  } else {
    lb = (int)((uint32_t)pos / (uint32_t)g.block_size);
    off = pos - lb * g.block_size;
  }
  lb = lb < table_len ? lb : table_len - 1;
  int phys = table[lb];
  phys = phys < 0 ? 0 : (phys >= g.num_blocks ? g.num_blocks - 1 : phys);
  return g.layer_offset + ((int64_t)phys * g.block_size + off) * g.row_elems;
}

// Caches kTableWindow consecutive block-table entries of one sequence in
// two VGPRs (entry base+i in lane i of the first, base+64+i of the second),
// so the per-tile physical-block lookup is a v_readlane instead of a memory
// load whose wait would also drain the prefetched K/V loads.
constexpr int kTableWindow = 2 * kWave;

struct TableCache {
  int base;        // first cached logical block (wave-uniform)
  int entries[2];  // lane i: table[base + i], table[base + 64 + i] (the row's last entry past its end)

  // The reads are clamped to the row's last entry (table_len >= 1), so they
  // need neither a branch nor a wait where they are issued; every lookup
  // asks for a block inside the row, so the entries past it are never used.
  __device__ __forceinline__ void load(const int32_t* table, int table_len, int first) {
    base = __builtin_amdgcn_readfirstlane(first);
    const int i = base + lane_id();
    entries[0] = table[min(i, table_len - 1)];
    entries[1] = table[min(i + kWave, table_len - 1)];
  }
  // Physical block of logical block `lb` (wave-uniform).  With kRefill the
  // window moves when `lb` leaves it; without, the caller guarantees
  // base <= lb < base + kTableWindow (no load inside the caller's loop, so
  // the compiler can keep counting that loop's outstanding K/V loads exactly).
  template <bool kRefill>
  __device__ __forceinline__ int lookup(const int32_t* table, int table_len, int lb) {
    lb = __builtin_amdgcn_readfirstlane(lb);
    if constexpr (kRefill) {
      if (lb < base || lb - base >= kTableWindow) load(table, table_len, lb);
    }
    int idx = lb - base;
    idx = idx < 0 ? 0 : (idx >= kTableWindow ? kTableWindow - 1 : idx);
    const int lo = __builtin_amdgcn_readlane(entries[0], idx & (kWave - 1));
    const int hi = __builtin_amdgcn_readlane(entries[1], idx & (kWave - 1));
    return idx < kWave ? lo : hi;
  }
};

// kWindows consecutive windows of kTableWindow block-table entries, loaded
// together (lane i of register r holds entry base + 64r + i), for a wave
// whose lookups only move forward: the front window serves the lookups, and
// when one passes it the queued windows move up a place (register moves, no
// load).  A prefill piece of up to kWindows x kTableWindow blocks so keeps
// its table in registers with no load inside its DMA loop, whose waits count
// the loop's outstanding K/V loads exactly.  (The moves sit behind a
// uniform branch in that loop, which cost the short pieces of a causal
// prompt about 6% when every lookup checked every window, so pieces that
// fit one window run the kWindows = 1 kernel, which has neither.)
template <int kWindows>
struct TableWindows {
  int base;                    // first logical block of the front window (wave-uniform)
  int entries[2 * kWindows];   // clamped to the row's last entry past its end

  // Only the registers that blocks [first, first + count) reach are loaded
  // (count wave-uniform; the others are never looked up).
  __device__ __forceinline__ void load(const int32_t* table, int table_len, int first, int count) {
    base = __builtin_amdgcn_readfirstlane(first);
    count = __builtin_amdgcn_readfirstlane(count);
#pragma unroll
    for (int r = 0; r < 2 * kWindows; ++r) {
      if (r < 2 || r * kWave < count) entries[r] = table[min(base + r * kWave + lane_id(), table_len - 1)];
    }
  }
  // Physical block of logical block `lb` (wave-uniform; lb never below an
  // earlier lookup's, less than two windows past the front window's first
  // block (a prefill wave's lookups advance a few blocks per step), and
  // below the first block + kWindows x kTableWindow).
  __device__ __forceinline__ int lookup_forward(int lb) {
    lb = __builtin_amdgcn_readfirstlane(lb);
    if (kWindows > 1 && lb - base >= kTableWindow) {  // uniform, once per window
#pragma unroll
      for (int r = 0; r + 2 < 2 * kWindows; ++r) entries[r] = entries[r + 2];
      base += kTableWindow;
    }
    int idx = lb - base;
    idx = idx < 0 ? 0 : (idx >= kTableWindow ? kTableWindow - 1 : idx);
    const int lo = __builtin_amdgcn_readlane(entries[0], idx & (kWave - 1));
    const int hi = __builtin_amdgcn_readlane(entries[1], idx & (kWave - 1));
    return idx < kWave ? lo : hi;
  }
};

// Addressing of the 16 keys of one tile (tiles start at multiples of 16).
// kUniform: block_size is a power of two >= 16, so the whole tile lies in one
// physical block: one wave-uniform lookup (through a TableCache) serves all
// lanes and per-lane offsets are 32-bit.  Otherwise every lane resolves its
// own key through the table.
template <bool kUniform, bool kRefill>
struct TileAddr {
  int64_t base;
  __device__ __forceinline__ void init(const CacheGeom& g, const int32_t* table, int table_len,
                                       TableCache& tc, int key0) {
    if constexpr (kUniform) {
      // uniform mode implies a power-of-two block size (see the launchers)
      key0 = __builtin_amdgcn_readfirstlane(key0);
      int lb = key0 >> g.bs_shift;
      const int off = key0 & (g.block_size - 1);
      lb = lb < table_len ? lb : table_len - 1;
      int phys = tc.template lookup<kRefill>(table, table_len, lb);
      phys = phys < 0 ? 0 : (phys >= g.num_blocks ? g.num_blocks - 1 : phys);
      base = g.layer_offset + ((int64_t)phys * g.block_size + off) * g.row_elems;
    }
  }
  // offset of key key0 + r
  __device__ __forceinline__ int64_t at(const CacheGeom& g, const int32_t* table, int table_len,
                                        int key0, int r) const {
    if constexpr (kUniform) {
      return base + (int64_t)(r * g.row_elems32);
    } else {
      return token_offset(g, table, table_len, key0 + r);
    }
  }
};

// ---------------------------------------------------------------------------
// MFMA tile math shared by decode and prefill
// ---------------------------------------------------------------------------
// Each lane holds, for its row (l%16: the key for K, the query row for Q),
// kVec 16-byte vectors; vector j covers bytes [64j + 16*(l/16), +16) of the
// row, so one load instruction reads 64 contiguous bytes of 16 rows.  The
// MFMA K index is mapped onto those dims identically for both operands, so
// the sum over all MFMAs is the full q.k dot product.
template <typename T, int D>
struct Frag {
  static constexpr int kBytes = D * Elt<T>::kBytes / 4;  // bytes of one lane's slice
  static constexpr int kVec = kBytes / 16;               // 16-byte vectors per slice
  uint4 v[kVec];
};

// Loads this lane's slice of a row (`row` = element 0 of the row).
template <typename T, int D>
__device__ __forceinline__ void load_slice(Frag<T, D>& f, const void* row) {
  const unsigned char* p = reinterpret_cast<const unsigned char*>(row) + 16 * (lane_id() >> 4);
#pragma unroll
  for (int j = 0; j < Frag<T, D>::kVec; ++j) f.v[j] = *reinterpret_cast<const uint4*>(p + 64 * j);
}

template <typename T, int D>
__device__ __forceinline__ v4f qk_mfma(const Frag<T, D>& k, const Frag<T, D>& q) {
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  if constexpr (Elt<T>::kIsBf16) {
    // MFMA c takes 4 bf16 (two dwords) of the slice; c -> (vector c/2, half c%2)
    const uint32_t* kw = reinterpret_cast<const uint32_t*>(k.v);
    const uint32_t* qw = reinterpret_cast<const uint32_t*>(q.v);
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      const v4s a = __builtin_bit_cast(v4s, u32x2_t{kw[2 * c], kw[2 * c + 1]});
      const v4s b = __builtin_bit_cast(v4s, u32x2_t{qw[2 * c], qw[2 * c + 1]});
      acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, acc, 0, 0, 0);
    }
  } else {
    const float* kf = reinterpret_cast<const float*>(k.v);
    const float* qf = reinterpret_cast<const float*>(q.v);
#pragma unroll
    for (int c = 0; c < D / 4; ++c) {
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[c], qf[c], acc, 0, 0, 0);
    }
  }
  return acc;
}

// Online-softmax state of one lane: the O^T accumulator for its query row
// (o[c][i] = O[row][16c + 4*(l/16) + i]), the running max of the row (equal
// in all four lane groups) and this lane's partial denominator.
template <int D>
struct SoftmaxState {
  v4f o[D / 16];
  float m;
  float lsum;

  __device__ __forceinline__ void init() {
#pragma unroll
    for (int c = 0; c < D / 16; ++c) o[c] = v4f{0.f, 0.f, 0.f, 0.f};
    m = kNegInf;
    lsum = 0.f;
  }
};

// Scores -> probabilities for one 16-key tile.  `s` holds the scaled scores
// (-inf where masked) and is overwritten with exp(s - m_new); the state is
// rescaled to the new running max.
template <int D>
__device__ __forceinline__ void softmax_tile(SoftmaxState<D>& st, v4f& s) {
  float tmax = score_max(score_max(s[0], s[1]), score_max(s[2], s[3]));
  tmax = max_over_groups(tmax);
  const float m_new = score_max(st.m, tmax);
  // A row with nothing unmasked so far keeps m = -inf; use 0 as the
  // reference point so the exponentials below are exact zeros, not NaN.
  const float nref = (m_new == kNegInf) ? 0.f : -m_new * kLog2e;
  float tsum = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s[i] = fast_exp2(fmaf(s[i], kLog2e, nref));
    tsum += s[i];
  }
  // Rescale only when some row's maximum moved (alpha would be exactly 1
  // otherwise); the test is wave-uniform.
  if (__ballot(m_new != st.m)) {
    const float alpha = fast_exp2(fmaf(st.m, kLog2e, nref));
    st.lsum = st.lsum * alpha + tsum;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) st.o[c] *= alpha;
  } else {
    st.lsum += tsum;
  }
  st.m = m_new;
}

// softmax_tile for kBlocks row blocks at once, with one (wave-uniform)
// rescale decision for all of them, so the blocks' chains interleave.
template <int D, int kBlocks>
__device__ __forceinline__ void softmax_tiles(SoftmaxState<D> (&st)[kBlocks], v4f (&s)[kBlocks]) {
  float m_new[kBlocks], nref[kBlocks], tsum[kBlocks];
  bool moved = false;
#pragma unroll
  for (int nb = 0; nb < kBlocks; ++nb) {
    const float tmax = max_over_groups(score_max(score_max(s[nb][0], s[nb][1]), score_max(s[nb][2], s[nb][3])));
    m_new[nb] = score_max(st[nb].m, tmax);
    nref[nb] = (m_new[nb] == kNegInf) ? 0.f : -m_new[nb] * kLog2e;
    tsum[nb] = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s[nb][i] = fast_exp2(fmaf(s[nb][i], kLog2e, nref[nb]));
      tsum[nb] += s[nb][i];
    }
    moved |= m_new[nb] != st[nb].m;
  }
  if (__ballot(moved)) {
#pragma unroll
    for (int nb = 0; nb < kBlocks; ++nb) {
      const float alpha = fast_exp2(fmaf(st[nb].m, kLog2e, nref[nb]));
      st[nb].lsum = st[nb].lsum * alpha + tsum[nb];
#pragma unroll
      for (int c = 0; c < D / 16; ++c) st[nb].o[c] *= alpha;
    }
  } else {
#pragma unroll
    for (int nb = 0; nb < kBlocks; ++nb) st[nb].lsum += tsum[nb];
  }
#pragma unroll
  for (int nb = 0; nb < kBlocks; ++nb) st[nb].m = m_new[nb];
}

// O^T += V^T . P^T for one 16-key tile.  `vt` is the LDS copy of the tile's
// V rows ([key][dim], row pitch `pitch` bytes); `p` holds this lane's four
// probabilities (keys 4*(l/16)+i of query row l%16).
template <typename T, int D>
__device__ __forceinline__ void pv_mfma(SoftmaxState<D>& st, const unsigned char* vt, int pitch,
                                        const v4f& p) {
  const int lane = lane_id();
  const int g = lane >> 4;
  const int col = lane & 15;
  if constexpr (Elt<T>::kIsBf16) {
    const v4s b = pack_bf16x4(p[0], p[1], p[2], p[3]);
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      v4s a;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint16_t* r = reinterpret_cast<const uint16_t*>(vt + (4 * g + e) * pitch);
        a[e] = (short)r[16 * c + col];
      }
      st.o[c] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, st.o[c], 0, 0, 0);
    }
  } else {
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float* r = reinterpret_cast<const float*>(vt + (4 * g + j) * pitch);
        st.o[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(r[16 * c + col], p[j], st.o[c], 0, 0, 0);
      }
    }
  }
}

// Scaled, dtype-rounded score (reference: einsum in the storage dtype, then
// `* scale` in the storage dtype).
template <typename T>
__device__ __forceinline__ float scaled_score(float acc, float scale) {
  return round_storage<T>(round_storage<T>(acc) * scale);
}

// Writes 4 consecutive output elements.
template <typename T>
__device__ __forceinline__ void store4(T* dst, float a, float b, float c, float d) {
  if constexpr (Elt<T>::kIsBf16) {
    uint2 w;
    w.x = pack_bf16x2(a, b);
    w.y = pack_bf16x2(c, d);
    *reinterpret_cast<uint2*>(dst) = w;
  } else {
    *reinterpret_cast<float4*>(dst) = make_float4(a, b, c, d);
  }
}

template <typename T>
__device__ __forceinline__ void store_elt(T* p, float x) {
  if constexpr (Elt<T>::kIsBf16) {
    reinterpret_cast<uint16_t*>(p)[0] = (uint16_t)f32_to_bf16_bits(x);
  } else {
    *reinterpret_cast<float*>(p) = x;
  }
}

// ---------------------------------------------------------------------------
// KV append / gather / block copy
// ---------------------------------------------------------------------------
__device__ __forceinline__ void copy_row(unsigned char* dst, const unsigned char* src,
                                         int64_t bytes, int vec_ok) {
  if (vec_ok) {
    for (int64_t i = threadIdx.x; i < bytes / 16; i += blockDim.x) {
      reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
    }
  } else {
    for (int64_t i = threadIdx.x; i < bytes / 2; i += blockDim.x) {
      reinterpret_cast<uint16_t*>(dst)[i] = reinterpret_cast<const uint16_t*>(src)[i];
    }
  }
}

// grid (num_tokens, 2): workgroup (t, 0) moves token t's K row, (t, 1) its V row.
__global__ __launch_bounds__(256) void kv_append_kernel(
    const unsigned char* __restrict__ k_new, int64_t k_stride_bytes,
    const unsigned char* __restrict__ v_new, int64_t v_stride_bytes,
    const int64_t* __restrict__ slots, int64_t num_tokens, unsigned char* __restrict__ k_cache,
    unsigned char* __restrict__ v_cache, int64_t layer_offset_bytes, int64_t num_slots,
    int64_t row_bytes, int vec_ok) {
  const int64_t t = blockIdx.x;
  if (t >= num_tokens) return;
  const int64_t slot = slots[t];
  if (slot < 0 || slot >= num_slots) return;
  const bool is_k = blockIdx.y == 0;
  const unsigned char* src = is_k ? k_new + t * k_stride_bytes : v_new + t * v_stride_bytes;
  unsigned char* dst = (is_k ? k_cache : v_cache) + layer_offset_bytes + slot * row_bytes;
  copy_row(dst, src, row_bytes, vec_ok);
}

// grid (token_count, 2)
__global__ __launch_bounds__(256) void kv_gather_kernel(
    const unsigned char* __restrict__ k_cache, const unsigned char* __restrict__ v_cache,
    int64_t layer_offset_bytes, int64_t num_blocks, int64_t block_size,
    const int32_t* __restrict__ table, int64_t table_len, int64_t token_count,
    unsigned char* __restrict__ k_out, unsigned char* __restrict__ v_out, int64_t row_bytes,
    int vec_ok) {
  const int64_t t = blockIdx.x;
  if (t >= token_count) return;
  int64_t lb = t / block_size;
  lb = lb < table_len ? lb : table_len - 1;
  int64_t phys = table[lb];
  phys = phys < 0 ? 0 : (phys >= num_blocks ? num_blocks - 1 : phys);
  const int64_t slot = phys * block_size + (t % block_size);
  const bool is_k = blockIdx.y == 0;
  const unsigned char* src = (is_k ? k_cache : v_cache) + layer_offset_bytes + slot * row_bytes;
  copy_row((is_k ? k_out : v_out) + t * row_bytes, src, row_bytes, vec_ok);
}

// grid (count, num_layers, 2): each workgroup moves one block of one layer.
__global__ __launch_bounds__(256) void kv_copy_blocks_kernel(
    const unsigned char* __restrict__ src_k, const unsigned char* __restrict__ src_v,
    int64_t src_num_blocks, const int32_t* __restrict__ src_blocks,
    unsigned char* __restrict__ dst_k, unsigned char* __restrict__ dst_v,
    int64_t dst_num_blocks, const int32_t* __restrict__ dst_blocks, int64_t count,
    int64_t block_bytes, int vec_ok) {
  const int64_t i = blockIdx.x;
  const int64_t layer = blockIdx.y;
  if (i >= count) return;
  int64_t sb = i, db = i, s_pool = count, d_pool = count;
  if (src_blocks != nullptr) {
    sb = src_blocks[i];
    s_pool = src_num_blocks;
  }
  if (dst_blocks != nullptr) {
    db = dst_blocks[i];
    d_pool = dst_num_blocks;
  }
  if (sb < 0 || sb >= s_pool || db < 0 || db >= d_pool) return;
  const bool is_k = blockIdx.z == 0;
  const unsigned char* src = (is_k ? src_k : src_v) + (layer * s_pool + sb) * block_bytes;
  unsigned char* dst = (is_k ? dst_k : dst_v) + (layer * d_pool + db) * block_bytes;
  copy_row(dst, src, block_bytes, vec_ok);
}

// ---------------------------------------------------------------------------
// Fused RoPE + KV append
// ---------------------------------------------------------------------------
// One grid row = one head of one token: rows t*(Hq + 2*Hkv) + j cover the q
// heads (j < Hq), then the k heads, then the v heads of token t.  A row takes
// D/2 lanes; lane i rotates the pair (x[i], x[i + D/2]) by the angle of
// frequency i at the token's position:
//     out[i]       = x[i]*cos - x[i+D/2]*sin
//     out[i + D/2] = x[i+D/2]*cos + x[i]*sin
// with every product and sum rounded to the storage dtype, as the
// reference's elementwise torch ops do (layers/rope.py:6-23), so the result
// is bit-identical to them given the same sin/cos rows.  q rows are rotated
// in place; rotated k rows and unrotated v rows go to the cache slot of the
// token (a negative or out-of-pool slot is skipped, as in kv_append).
struct RopeAppendArgs {
  void* q;
  int64_t q_st, q_sh;
  const void* k;
  int64_t k_st, k_sh;
  const void* v;
  int64_t v_st, v_sh;
  const int64_t* positions;
  const int64_t* slots;
  int64_t num_tokens;
  const void* cos_table;  // (table_rows, head_dim / 2)
  const void* sin_table;
  int64_t table_rows;
  void* k_cache;
  void* v_cache;
  int64_t layer_offset;  // elements before the layer
  int64_t pool_slots;    // num_blocks * block_size
  int32_t q_heads;
  int32_t kv_heads;
};

template <typename T>
__device__ __forceinline__ float load_elt(const void* base, int64_t i) {
  if constexpr (Elt<T>::kIsBf16) {
    return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(base)[i]);
  } else {
    return reinterpret_cast<const float*>(base)[i];
  }
}

// a*b and a+-b in the storage dtype, each rounded on its own: contraction
// into fused multiply-adds (hipcc's default) is switched off here, because
// the reference computes every product and sum as a separate torch op.
template <typename T>
__device__ __forceinline__ float mul_t(float a, float b) {
#pragma clang fp contract(off)
  return round_storage<T>(a * b);
}
template <typename T>
__device__ __forceinline__ float add_t(float a, float b) {
#pragma clang fp contract(off)
  return round_storage<T>(a + b);
}
template <typename T>
__device__ __forceinline__ float sub_t(float a, float b) {
#pragma clang fp contract(off)
  return round_storage<T>(a - b);
}

template <typename T, int D>
__global__ __launch_bounds__(256) void rope_kv_append_kernel(RopeAppendArgs a) {
  constexpr int kHalf = D / 2;
  constexpr int kRowsPerBlock = 256 / kHalf;
  const int sub = threadIdx.x / kHalf;
  const int i = threadIdx.x % kHalf;
  const int heads = a.q_heads + 2 * a.kv_heads;
  const int64_t r = (int64_t)blockIdx.x * kRowsPerBlock + sub;
  if (r >= a.num_tokens * heads) return;
  const int64_t t = r / heads;
  const int j = (int)(r - t * heads);
  int64_t pos = a.positions[t];
  pos = pos < 0 ? 0 : (pos >= a.table_rows ? a.table_rows - 1 : pos);
  const float c = load_elt<T>(a.cos_table, pos * kHalf + i);
  const float s = load_elt<T>(a.sin_table, pos * kHalf + i);
  if (j < a.q_heads) {
    T* x = reinterpret_cast<T*>(a.q) + t * a.q_st + (int64_t)j * a.q_sh;
    const float x1 = load_elt<T>(x, i);
    const float x2 = load_elt<T>(x, i + kHalf);
    store_elt<T>(x + i, sub_t<T>(mul_t<T>(x1, c), mul_t<T>(x2, s)));
    store_elt<T>(x + i + kHalf, add_t<T>(mul_t<T>(x2, c), mul_t<T>(x1, s)));
    return;
  }
  const int64_t slot = a.slots[t];
  if (slot < 0 || slot >= a.pool_slots) return;
  const bool is_k = j < a.q_heads + a.kv_heads;
  const int h = is_k ? j - a.q_heads : j - a.q_heads - a.kv_heads;
  const int64_t dst_off = a.layer_offset + (slot * a.kv_heads + h) * D;
  if (is_k) {
    const T* x = reinterpret_cast<const T*>(a.k) + t * a.k_st + (int64_t)h * a.k_sh;
    const float x1 = load_elt<T>(x, i);
    const float x2 = load_elt<T>(x, i + kHalf);
    T* dst = reinterpret_cast<T*>(a.k_cache) + dst_off;
    store_elt<T>(dst + i, sub_t<T>(mul_t<T>(x1, c), mul_t<T>(x2, s)));
    store_elt<T>(dst + i + kHalf, add_t<T>(mul_t<T>(x2, c), mul_t<T>(x1, s)));
  } else {
    const T* x = reinterpret_cast<const T*>(a.v) + t * a.v_st + (int64_t)h * a.v_sh;
    T* dst = reinterpret_cast<T*>(a.v_cache) + dst_off;
    dst[i] = x[i];
    dst[i + kHalf] = x[i + kHalf];
  }
}

// ---------------------------------------------------------------------------
// Greedy token selection: argmax of each logits row
// ---------------------------------------------------------------------------
// (value, index) pairs ordered like torch.argmax: a larger value wins, NaN
// beats every number, and equal values (or two NaNs) go to the lower index.
__device__ __forceinline__ bool argmax_better(float v, int64_t i, float bv, int64_t bi) {
  const bool vn = v != v;
  const bool bn = bv != bv;
  if (vn != bn) return vn;
  if (!vn && v != bv) return v > bv;
  return i < bi;
}

constexpr int kArgmaxThreads = 1024;

// (value, index) of a piece of a row, for nie_argmax_rows_split's second pass.
struct ArgmaxPartial {
  float value;
  int32_t pad;
  int64_t index;
};
constexpr int64_t kArgmaxPieceCols = 8192;  // one 16-byte bf16 vector per thread

// One workgroup per row (grid.y == 1), or per (row, piece of
// kArgmaxPieceCols columns) with `partial` set; each thread scans 16-byte
// vectors of its columns (a scalar tail covers rows whose length or start is
// not vector aligned), then the workgroup reduces (value, index) through LDS
// and writes the row's index, or the piece's pair to partial[row * grid.y +
// piece].
template <typename T>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_rows_kernel(const void* logits, int64_t row_stride,
                                                                     int64_t cols, int64_t* out,
                                                                     ArgmaxPartial* partial) {
  constexpr int kPerVec = 16 / Elt<T>::kBytes;
  const int64_t row = blockIdx.x;
  const T* x = reinterpret_cast<const T*>(logits) + row * row_stride;
  const int64_t c0 = partial != nullptr ? (int64_t)blockIdx.y * kArgmaxPieceCols : 0;
  const int64_t c1 = partial != nullptr && c0 + kArgmaxPieceCols < cols ? c0 + kArgmaxPieceCols : cols;
  float best = kNegInf;
  int64_t best_i = cols;  // past the end: loses every comparison with a real element
  const bool vec = ((uintptr_t)x % 16) == 0;
  const int64_t vec_end = vec ? c1 / kPerVec : 0;  // c0 is a multiple of kPerVec
  const int64_t nvec = vec ? cols / kPerVec : 0;
  for (int64_t j = c0 / kPerVec + threadIdx.x; j < vec_end; j += kArgmaxThreads) {
    const uint4 w = reinterpret_cast<const uint4*>(x)[j];
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < kPerVec; ++e) {
      float v;
      if constexpr (Elt<T>::kIsBf16) {
        v = bf16_bits_to_f32((words[e / 2] >> (16 * (e % 2))) & 0xffffu);
      } else {
        v = __uint_as_float(words[e]);
      }
      const int64_t i = j * kPerVec + e;
      if (argmax_better(v, i, best, best_i)) {
        best = v;
        best_i = i;
      }
    }
  }
  for (int64_t i = (nvec * kPerVec > c0 ? nvec * kPerVec : c0) + threadIdx.x; i < c1; i += kArgmaxThreads) {
    const float v = load_elt<T>(x, i);
    if (argmax_better(v, i, best, best_i)) {
      best = v;
      best_i = i;
    }
  }
  // wave reduction, then one pair per wave through LDS
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float v = __shfl_xor(best, off);
    const int64_t i = __shfl_xor(best_i, off);
    if (argmax_better(v, i, best, best_i)) {
      best = v;
      best_i = i;
    }
  }
  __shared__ float s_val[kArgmaxThreads / kWave];
  __shared__ int64_t s_idx[kArgmaxThreads / kWave];
  const int wave = threadIdx.x / kWave;
  if (lane_id() == 0) {
    s_val[wave] = best;
    s_idx[wave] = best_i;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kArgmaxThreads / kWave; ++w) {
      if (argmax_better(s_val[w], s_idx[w], best, best_i)) {
        best = s_val[w];
        best_i = s_idx[w];
      }
    }
    if (partial != nullptr) {
      partial[row * gridDim.y + blockIdx.y] = ArgmaxPartial{best, 0, best_i};
    } else {
      out[row] = best_i;
    }
  }
}

// Second pass of nie_argmax_rows_split: one wave per row over its pieces'
// pairs (argmax_better is a strict total order, so the pieces' order of
// combination does not change the result).
__global__ __launch_bounds__(kWave) void argmax_merge_kernel(const ArgmaxPartial* partial, int64_t pieces,
                                                             int64_t* out) {
  const int64_t row = blockIdx.x;
  float best = kNegInf;
  int64_t best_i = INT64_MAX;
  for (int64_t p = lane_id(); p < pieces; p += kWave) {
    const ArgmaxPartial q = partial[row * pieces + p];
    if (argmax_better(q.value, q.index, best, best_i)) {
      best = q.value;
      best_i = q.index;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float v = __shfl_xor(best, off);
    const int64_t i = __shfl_xor(best_i, off);
    if (argmax_better(v, i, best, best_i)) {
      best = v;
      best_i = i;
    }
  }
  if (lane_id() == 0) out[row] = best_i;
}

// ---------------------------------------------------------------------------
// Paged decode (split-K)
// ---------------------------------------------------------------------------
constexpr int kDecodeWaves = 8;  // KV heads handled by one workgroup (one per wave)

// Control region at the start of every decode and prefill workspace: one
// counter per (sequence, KV head) of a call, for the one-launch
// decode's splits to find each other (decode_fused_kernel), each on a
// 128-byte line of its own (the pollers of different counters do not meet
// on one line), and a count of the waits that gave up.  It must be zero
// before a workspace's first call; every call leaves the counters zero
// again.
constexpr int64_t kCtlBytes = 256 * 1024;
constexpr int kCtlSlotBytes = 128;
constexpr int kCtlPairs = (int)(kCtlBytes / kCtlSlotBytes) - 1;

struct DecodeCtlSlot {
  uint32_t count;  // splits of the pair that have published their (max, sum) pairs
  uint32_t done;   // splits of the pair that have published their output shares
  uint32_t pad[kCtlSlotBytes / 4 - 2];
};

struct DecodeCtl {
  DecodeCtlSlot pair[kCtlPairs];
  DecodeCtlSlot gave_up;  // .count: waits that gave up (only grows; a diagnostic count)
};
static_assert(sizeof(DecodeCtl) == kCtlBytes, "control words fill their region");

struct DecodeArgs {
  const void* q;
  int64_t q_sb, q_sh;
  const void* k_cache;
  const void* v_cache;
  CacheGeom geom;
  int32_t q_heads;
  int32_t group;  // q_heads / kv_heads
  const int32_t* tables;
  int64_t table_stride;
  const int32_t* seq_lens;
  int64_t batch;
  int32_t tiles_per_split;  // 16-key tiles per work item; 0: derived on the device from the lengths
  int32_t split_slots;      // with tiles_per_split 0: workgroups the device plan aims to fill
  float scale;
  void* out;
  int64_t o_sb, o_sh;
  float* ws_o;   // (ws_items, q_heads, head_dim)
  float* ws_ml;  // (ws_items, q_heads, 2)
  int64_t ws_items;  // partial slots in the workspace (0 when there is none)
  // Two-pass rounding: the scores, (ws_items, tiles_per_split, q_heads, 16)
  // bf16, written by the scores pass and read by the P.V pass
  uint16_t* ws_s = nullptr;
  int64_t ws_s_keys = 0;  // key slots there (items x tiles_per_split x 16 must fit)
  // Fused append (nie_paged_decode_append): new K/V rows (batch, kv_heads,
  // head_dim), row strides in elements; k_new == nullptr: no append.
  const void* k_new = nullptr;
  const void* v_new = nullptr;
  int64_t kn_s = 0, vn_s = 0;
  // RoPE of q and of the new K rows at position seq_len - 1 (fused append
  // only): cos / sin tables (rope_rows, head_dim / 2); nullptr: none
  const void* rope_cos = nullptr;
  const void* rope_sin = nullptr;
  int64_t rope_rows = 0;
  // A work-item table in device memory (nie_paged_decode_append_planned): a
  // captured launch replays with the plan its step's host lengths call for,
  // written there before each replay; count 0 there: locate on the device.
  const struct DecodeItems* __restrict__ dev_items = nullptr;
  // One-launch decode: the workspace's control region, and the polls a
  // split's wait for the others makes before it forms their statistics
  // itself
  DecodeCtl* ctl = nullptr;
  int32_t spin_limit = 0;
  // One-pass rounding: the split that finishes last merges the partials of
  // its (sequence, KV head), counted on ctl's counters (no merge launch)
  int32_t merge_last = 0;
};

// Work items of a decode call planned from host copies of the lengths,
// passed by value as a kernel argument (or read from device memory, see
// DecodeArgs::dev_items): item i = sequence << 16 | split, the split length
// in 16-key tiles, and per sequence its length and first item.  count 0:
// the kernels locate their work from the device lengths instead.
constexpr int kMaxDecodeItems = 256;
constexpr int kMaxDecodeSeqs = 128;

struct DecodeItems {
  int32_t count;
  int32_t tps;
  uint32_t item[kMaxDecodeItems];
  int32_t seq_len[kMaxDecodeSeqs];
  int32_t seq_first[kMaxDecodeSeqs];
};

// Split length of a call planned on the device: the smallest number of
// 16-key tiles per work item (within [kDecodeMinTilesPerSplit,
// kDecodeMaxTilesPerSplit]) whose items fit `slots` workgroups in one round.
// With `tiles` = sum over the sequences of ceil(len / 16), a call then has
// at most tiles / tps + batch <= slots - 1 items unless the upper clamp binds.
constexpr int64_t kDecodeMinTilesPerSplit = 2;
constexpr int64_t kDecodeMaxTilesPerSplit = 2 * kWave;  // the per-split block-table window

__host__ __device__ inline int64_t decode_device_tps(int64_t tiles, int64_t batch, int64_t slots) {
  const int64_t room = slots - batch - 1;
  int64_t tps = room > 0 ? cdiv(tiles, room) : kDecodeMaxTilesPerSplit;
  tps = tps < kDecodeMinTilesPerSplit ? kDecodeMinTilesPerSplit : tps;
  return tps > kDecodeMaxTilesPerSplit ? kDecodeMaxTilesPerSplit : tps;
}

__device__ __forceinline__ int64_t wave_sum64(int64_t x) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) x += __shfl_xor(x, off);
  return x;
}

// The split length of a decode call: the host's, or (tiles_per_split 0) the
// device plan's from the lengths themselves; wave-uniform.  first_len gets
// this lane's length of the first 64 sequences (those every caller reads).
__device__ __forceinline__ int64_t decode_call_tps(const DecodeArgs& a, int* first_len) {
  const int lane = lane_id();
  *first_len = lane < a.batch ? a.seq_lens[lane] : 0;
  if (a.tiles_per_split > 0) return a.tiles_per_split;
  int64_t tiles = *first_len > 0 ? cdiv((int64_t)*first_len, (int64_t)kTileKeys) : 0;
  for (int64_t b = kWave + lane; b < a.batch; b += kWave) {
    const int64_t len = a.seq_lens[b];
    tiles += len > 0 ? cdiv(len, (int64_t)kTileKeys) : 0;
  }
  return uniform64(decode_device_tps(wave_sum64(tiles), a.batch, a.split_slots));
}

// Items of sequence b of a call with split length tps (first_len: the
// calling lane's length when b is that lane's sequence among the first 64).
__device__ __forceinline__ int64_t decode_splits_of(const DecodeArgs& a, int64_t b, int64_t tps, int first_len) {
  const int64_t len = b == lane_id() ? first_len : a.seq_lens[b];
  return len > 0 ? cdiv(cdiv(len, (int64_t)kTileKeys), tps) : (int64_t)0;
}

// s_waitcnt immediate that waits until at most `n` vector-memory operations
// are outstanding and leaves the export / LGKM counters alone (gfx9 encoding).
constexpr int waitcnt_vm(int n) { return (n & 0xf) | ((n >> 4) << 14) | (0x7 << 4) | (0xf << 8); }

// Waits until at most `later` groups of kOps vector-memory operations are
// outstanding: the DMA ops of the tiles (or key steps) a ring pipeline has
// issued after the one about to be read.  `later` is wave-uniform and at
// most kMaxLater; the ring issues only tiles that exist, so near the end of
// an item fewer groups are in flight and the wait tightens with them.
template <int kOps, int kMaxLater>
__device__ __forceinline__ void wait_dma_groups(int later) {
  static_assert(kMaxLater >= 0 && kMaxLater <= 7 && kMaxLater * kOps < 64, "vmcnt immediate range");
  if constexpr (kMaxLater >= 1) {
    // s_waitcnt takes an immediate: one test per possible group count,
    // from the most groups down (a count above kMaxLater waits for kMaxLater)
    if (later >= kMaxLater) {
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(kMaxLater * kOps));
      return;
    }
    wait_dma_groups<kOps, kMaxLater - 1>(later);
  } else {
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  }
}

typedef __attribute__((address_space(3))) void lds_void_t;

// Cache policy of a DMA read: kCacheDefault, or kCacheStream (the `nt` bit),
// which marks the lines as streaming.  A plain 1 GiB read through
// global_load_lds_dwordx4 sustains 6.2 TB/s on MI355X with the default policy
// and 7.0 TB/s with nt, at 256 to 1024 workgroups.
constexpr int kCacheDefault = 0;
constexpr int kCacheStream = 2;
// Prefill re-reads a chunk's context tiles once per query tile, so its K/V
// reads keep the default policy.
constexpr int kPrefillCachePolicy = kCacheDefault;

// 16-byte-per-lane global -> LDS DMA (global_load_lds_dwordx4): lane l's 16
// bytes land at dst + 16*l.  The builtin exists only in the device pass; in
// the host pass (which only emits launch stubs) it would make clang drop the
// enclosing kernel's stub, so the host pass sees an empty body.
template <int kPolicy = kCacheDefault>
__device__ __forceinline__ void lds_dma16(const void* src, unsigned char* dst) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(src, (lds_void_t*)dst, 16, 0, kPolicy);
#else
  (void)src;
  (void)dst;
#endif
}

// ---------------------------------------------------------------------------
// Decode staging.  A workgroup owns a group of kHeads KV heads (one wave per
// head) and, for every 16-key tile, stages in LDS the K and V rows of all its
// heads: row r of a tile is key key0+r's contiguous slice of kHeads*D
// elements (1 KiB for 8 bf16 heads of 64 dims).  The rows are fetched with
// LDS DMA (global_load_lds_dwordx4), 64 lanes x 16 bytes = 1 KiB of
// consecutive bytes per op, spread round-robin over the waves, so every op
// is a fully contiguous read — the access pattern of a streaming copy.
// Chunk c of row r is stored at chunk position c ^ (r & 15): the MFMA K
// reads (16 lanes read one chunk of 16 different rows) hit distinct LDS
// banks, and the transposing V^T reads (16 rows x two adjacent chunks) spread
// over all 16 bank groups, two chunks each.
// ---------------------------------------------------------------------------
template <typename T, int D, int kHeads>
struct GroupTile {
  static constexpr int kSliceBytes = kHeads * D * Elt<T>::kBytes;  // one key's row
  static constexpr int kChunks = kSliceBytes / 16;                  // 16-byte chunks per row
  static constexpr int kSwzMask = (kChunks < 16 ? kChunks : 16) - 1;
  static constexpr int kBytes = kTileKeys * kSliceBytes;           // one K (or V) tile
  static constexpr int kOps = kBytes / (kWave * 16);               // DMA ops per K (or V) tile
  static constexpr int kRowsPerOp = kWave * 16 / kSliceBytes;
  static constexpr int kOpsPerWave = kOps / kHeads;
  static_assert(kSliceBytes <= kWave * 16 && (kWave * 16) % kSliceBytes == 0, "slice must divide 1 KiB");
  static_assert(kOps % kHeads == 0, "ops must spread evenly over the waves");
  __device__ static __forceinline__ int swz(int r) { return r & kSwzMask; }
  // LDS byte offset of 16-byte chunk c of row r
  __device__ static __forceinline__ int chunk_offset(int r, int c) { return r * kSliceBytes + ((c ^ swz(r)) << 4); }
  // LDS byte offset of element d of head hl in row r
  __device__ static __forceinline__ int elt_offset(int r, int hl, int d) {
    const int byte = (hl * D + d) * Elt<T>::kBytes;
    return chunk_offset(r, byte >> 4) + (byte & 15);
  }
  // This lane's transposing-read address (relative to the V tile) for the
  // V^T operand of dims 16c..16c+15 of head hl (see ring_read_vt4).
  __device__ static __forceinline__ int vt_offset(int lane, int hl, int c) {
    return elt_offset(4 * (lane >> 4) + ((lane >> 2) & 3), hl, 16 * c + 4 * (lane & 3));
  }
};

// ---------------------------------------------------------------------------
// Ring reads.  The tiles arrive by LDS DMA, whose destination the compiler
// cannot tell apart per ring slot, so compiler-visible LDS reads of the ring
// would each be preceded by a wait for *all* DMA in flight.  The bf16 path
// therefore reads the ring with inline-asm ds_reads, after the explicit
// vmcnt wait + barrier that cover exactly the tile being read; a closing
// lgkmcnt(0) asm takes every result as a read-write operand, so no use of a
// result can be scheduled before the data has arrived.
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t lds_off(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// kVec 16-byte K chunks (MFMA A layout) at precomputed LDS addresses.
template <int kVec>
__device__ __forceinline__ void ring_read_k(uint4 (&out)[kVec], const uint32_t (&addr)[kVec]) {
  v4u r[kVec];
#pragma unroll
  for (int j = 0; j < kVec; ++j) asm volatile("ds_read_b128 %0, %1" : "=v"(r[j]) : "v"(addr[j]));
  if constexpr (kVec == 2) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(r[0]), "+v"(r[1]));
  } else if constexpr (kVec == 4) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]));
  } else {
    static_assert(kVec == 8, "2, 4 or 8 chunks");
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]));
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(r[4]), "+v"(r[5]), "+v"(r[6]), "+v"(r[7]));
  }
#pragma unroll
  for (int j = 0; j < kVec; ++j) out[j] = uint4{r[j][0], r[j][1], r[j][2], r[j][3]};
}

// Four bf16 V^T MFMA A operands (16 dims x 16 keys each), one transposing
// LDS read each (ds_read_b64_tr_b16).  Within each group of 16 lanes the
// read transposes a 4 x 16 block: lane 16a + 4e + c supplies the address of
// four consecutive dims 4c..4c+3 of key 4a + e, and lane 16a + m receives
// dim m of keys 4a..4a+3 — the A layout of v_mfma_f32_16x16x16_bf16 for
// V^T (row = dim, k = key).  vt_offset() gives those per-lane addresses.
typedef unsigned v2u __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void ring_read_vt4(v4s (&a)[4], const uint32_t (&addr)[4]) {
  v2u r[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r[i]) : "v"(addr[i]));
  asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]));
#pragma unroll
  for (int c = 0; c < 4; ++c) a[c] = __builtin_bit_cast(v4s, r[c]);
}

// ---------------------------------------------------------------------------
// Decoder-layer elementwise work on either side of attention
// ---------------------------------------------------------------------------
constexpr int kNormThreads = 256;
constexpr int kNormVecsPerThread = 4;  // cols <= 256 x 4 x (16 bytes / element size)

// Element e of a 16-byte vector of T as float.
template <typename T>
__device__ __forceinline__ float vec_elt(const v4u& w, int e) {
  if constexpr (Elt<T>::kIsBf16) {
    return bf16_bits_to_f32((w[e / 2] >> (16 * (e % 2))) & 0xffffu);
  } else {
    return __uint_as_float(w[e]);
  }
}

// RMSNorm of one row per workgroup, in the arithmetic of the reference's
// RmsNorm.forward (layers/rms_norm.py:25-31): h = fp32(x),
// h / sqrt(mean(h * h) + eps), times fp32(weight), cast to the storage dtype
// (round to nearest even).  Only the order of the sum of squares differs from
// torch's reduction.  With `res`, the row is first x + res rounded to the
// storage dtype (the decoder's residual add, layers/decoder.py:50-51), which
// also goes to sum_out.  Each thread keeps its (up to kNormVecsPerThread)
// 16-byte vectors in registers between the two passes.
template <typename T>
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(const void* x, int64_t x_stride, const void* res,
                                                              int64_t res_stride, void* sum_out,
                                                              int64_t sum_stride, const void* weight, void* out,
                                                              int64_t out_stride, int cols, float eps) {
  constexpr int kPerVec = 16 / Elt<T>::kBytes;
  const int64_t row = blockIdx.x;
  const int nvec = cols / kPerVec;
  const v4u* xr = reinterpret_cast<const v4u*>(reinterpret_cast<const T*>(x) + row * x_stride);
  v4u v[kNormVecsPerThread];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kNormVecsPerThread; ++k) {
    const int j = (int)threadIdx.x + k * kNormThreads;
    if (j >= nvec) break;
    v[k] = xr[j];
    if (res != nullptr) {
      const v4u r = reinterpret_cast<const v4u*>(reinterpret_cast<const T*>(res) + row * res_stride)[j];
      v4u sum;
      if constexpr (Elt<T>::kIsBf16) {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          sum[w] = pack_bf16x2(vec_elt<T>(v[k], 2 * w) + vec_elt<T>(r, 2 * w),
                               vec_elt<T>(v[k], 2 * w + 1) + vec_elt<T>(r, 2 * w + 1));
        }
      } else {
#pragma unroll
        for (int w = 0; w < 4; ++w) sum[w] = __float_as_uint(vec_elt<T>(v[k], w) + vec_elt<T>(r, w));
      }
      v[k] = sum;
      reinterpret_cast<v4u*>(reinterpret_cast<T*>(sum_out) + row * sum_stride)[j] = sum;
    }
#pragma unroll
    for (int e = 0; e < kPerVec; ++e) {
      const float h = vec_elt<T>(v[k], e);
      ss = fmaf(h, h, ss);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  __shared__ float s_ss[kNormThreads / kWave];
  if (lane_id() == 0) s_ss[threadIdx.x / kWave] = ss;
  __syncthreads();
  ss = 0.f;
#pragma unroll
  for (int w = 0; w < kNormThreads / kWave; ++w) ss += s_ss[w];
  const float denom = sqrtf(ss * (1.f / (float)cols) + eps);
  v4u* orow = reinterpret_cast<v4u*>(reinterpret_cast<T*>(out) + row * out_stride);
  const v4u* wv = reinterpret_cast<const v4u*>(weight);
#pragma unroll
  for (int k = 0; k < kNormVecsPerThread; ++k) {
    const int j = (int)threadIdx.x + k * kNormThreads;
    if (j >= nvec) break;
    const v4u wk = weight != nullptr ? wv[j] : v4u{0u, 0u, 0u, 0u};
    float y[kPerVec];
#pragma unroll
    for (int e = 0; e < kPerVec; ++e) {
      y[e] = vec_elt<T>(v[k], e) / denom;
      if (weight != nullptr) y[e] = vec_elt<T>(wk, e) * y[e];
    }
    v4u o;
    if constexpr (Elt<T>::kIsBf16) {
#pragma unroll
      for (int w = 0; w < 4; ++w) o[w] = pack_bf16x2(y[2 * w], y[2 * w + 1]);
    } else {
#pragma unroll
      for (int w = 0; w < 4; ++w) o[w] = __float_as_uint(y[w]);
    }
    orow[j] = o;
  }
}

// SwiGLU's product silu(gate) * up (layers/mlp.py:18-22) as torch computes
// it in two kernels: s = silu(gate) in fp32, x / (1 + exp(-x)), rounded to
// the storage dtype, then s * up in fp32, rounded again.  Rows of `cols`
// elements at element strides (gate and up may be the two halves of one
// fused projection's output); one 16-byte vector per thread.
template <typename T>
__global__ __launch_bounds__(256) void silu_mul_kernel(const void* gate, int64_t gate_stride, const void* up,
                                                       int64_t up_stride, void* out, int64_t out_stride,
                                                       int64_t vecs_per_row, int64_t nvec) {
  constexpr int kPerVec = 16 / Elt<T>::kBytes;
  const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (j >= nvec) return;
  const int64_t r = j / vecs_per_row;
  const int64_t c = (j - r * vecs_per_row) * kPerVec;
  const v4u g = *reinterpret_cast<const v4u*>(reinterpret_cast<const T*>(gate) + r * gate_stride + c);
  const v4u u = *reinterpret_cast<const v4u*>(reinterpret_cast<const T*>(up) + r * up_stride + c);
  float y[kPerVec];
#pragma unroll
  for (int e = 0; e < kPerVec; ++e) {
    const float a = vec_elt<T>(g, e);
    float sl = a / (1.f + expf(-a));
    if constexpr (Elt<T>::kIsBf16) sl = bf16_bits_to_f32(f32_to_bf16_bits(sl));
    y[e] = sl * vec_elt<T>(u, e);
  }
  v4u o;
  if constexpr (Elt<T>::kIsBf16) {
#pragma unroll
    for (int w = 0; w < 4; ++w) o[w] = pack_bf16x2(y[2 * w], y[2 * w + 1]);
  } else {
#pragma unroll
    for (int w = 0; w < 4; ++w) o[w] = __float_as_uint(y[w]);
  }
  *reinterpret_cast<v4u*>(reinterpret_cast<T*>(out) + r * out_stride + c) = o;
}

// ---------------------------------------------------------------------------
// Decode-step projections: y = x . W^T over at most 16 rows (bf16)
// ---------------------------------------------------------------------------
// A decode step multiplies at most one row per sequence by each weight, so
// these GEMMs stream their weights once and are HBM-bound: 2*N*K bytes for
// 2*rows*N*K flops.  The work is tiles of 16 output columns (the SwiGLU
// epilogue: 16 gate rows and the 16 matching up rows of the weight), each
// walked in passes of 16 weight rows x 1024 k (32 KiB).  One workgroup per
// CU streams the passes of its tiles (tile blockIdx.x, then + gridDim.x, ...)
// through a 4-stage LDS ring, three passes in flight while one is multiplied:
//  - each wave of eight DMAs 2 of the 16 rows of a pass with global_load_lds_dwordx4
//    (one op = 1 KiB of one row, contiguous) under the non-temporal policy
//    (every weight byte is read once);
//  - a row's 16-byte slot S sits at LDS slot S ^ (row & 15), so the MFMA
//    operand reads (16 rows, the same k) hit 16 different bank groups;
//  - wave w multiplies the k eighth w of each pass: per 32-wide chunk one
//    v_mfma_f32_16x16x32_bf16 with x as the A operand (row l%16, k
//    8*(l/16)..+7) and the weight rows as B (column l%16, the same k).  A
//    wave loads its x operands of the whole k into registers once (x is
//    read by every workgroup: the L2 serves it);
//  - at a tile's last pass the eight waves' sums meet in LDS and wave 0
//    writes the tile while the ring keeps streaming.
// Epilogues: kLinearPlain writes bf16(x . W^T).  kLinearSiluMul alternates
// gate and up passes over the same k range and writes silu(gate) * up with
// torch's roundings: gate and up rounded to bf16 (the GEMM outputs), silu in
// fp32 rounded, the product rounded (layers/mlp.py:18-22 of the reference
// engine; nie_silu_mul's arithmetic).
constexpr int kLinearWaves = 8;
constexpr int kLinearMaxRows = 16;
constexpr int kLinearPassBytes = 32 * 1024;
constexpr int kLinearStages = 4;
constexpr int kLinearPlain = 0;
constexpr int kLinearSiluMul = 1;
constexpr int kLinearNoNorm = 0;
constexpr int kLinearNorm = 1;
constexpr int kLinearNormRes = 2;

struct LinearArgs {
  const bf16_t* x;
  int64_t x_stride;  // elements between rows of x
  int32_t rows;      // 1..16
  const bf16_t* w;   // (n, k) row-major; (2n, k) for kLinearSiluMul
  int64_t n;         // output columns
  int64_t k;
  bf16_t* y;
  int64_t y_stride;
  // RMSNorm folded into the x operand (the kNorm kernels): x is replaced by
  // norm_w * (h / sqrt(mean(h*h) + eps)), h = x + res (res may be null),
  // and workgroup 0 writes h to sum_out when both are given
  const bf16_t* res;
  int64_t res_stride;
  bf16_t* sum_out;
  int64_t sum_stride;
  const bf16_t* norm_w;
  float eps;
};

__device__ __forceinline__ bf16x8_t load_bf16x8(const bf16_t* p) {
  return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const v4u*>(p));
}

// f(integral_constant<int, I>) for I = kBegin .. kEnd - 1.
template <int kBegin, int kEnd, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (kBegin < kEnd) {
    f(std::integral_constant<int, kBegin>{});
    static_for<kBegin + 1, kEnd>(f);
  }
}

// kKPasses = k / 1024 (2, 4 or 8; 2 with a norm); grid.x <= the number of tiles.
// kNorm: kLinearNoNorm, kLinearNorm (RMSNorm of x) or kLinearNormRes (of x + res).
template <int kEpi, int kKPasses, int kNorm>
__global__ __launch_bounds__(kLinearWaves* kWave) void linear_rows_kernel(LinearArgs a) {
  constexpr int kSets = kEpi == kLinearSiluMul ? 2 : 1;
  constexpr int kPasses = kSets * kKPasses;             // passes per tile
  constexpr int kRowBytes = kLinearPassBytes / 16;      // 2 KiB of each row per pass
  constexpr int kPassK = kRowBytes / 2;                 // 1024
  constexpr int kPieces = kRowBytes / (kWave * 16);     // 2 DMA ops per row and pass
  constexpr int kRowsPerWave = 16 / kLinearWaves;       // 2
  constexpr int kOps = kRowsPerWave * kPieces;          // DMA ops per wave and pass
  constexpr int kWaveK = kPassK / kLinearWaves;         // 128
  constexpr int kChunks = kWaveK / 32;                  // 4 MFMAs per wave and pass
  // passes per loop trip: stage (q % 4) and pass (q % kPasses) of every step
  // are then compile-time constants
  constexpr int kTrip = kPasses > kLinearStages ? kPasses : kLinearStages;
  static_assert(kTrip % kPasses == 0 && kTrip % kLinearStages == 0, "trip covers whole tiles and ring turns");
  static_assert(kNorm == kLinearNoNorm || kKPasses == 2, "the folded RMSNorm is built for k = 2048");
  __shared__ __attribute__((aligned(16))) unsigned char ring[kLinearStages][kLinearPassBytes];
  __shared__ v4f red[kSets][kLinearWaves][kWave];
  // the folded norm's row totals; its per-vector partial sums of squares
  // (16 rows x k/8 vectors, 16 KiB) use ring stage 3, which the first pass
  // to fill it (pass 3, issued after the prologue's last barrier) finds free
  __shared__ float norm_ss[16];
  constexpr int kNormVecs = kKPasses * kPassK / 8;
  static_assert(kNorm == kLinearNoNorm || 16 * kNormVecs * 4 <= kLinearPassBytes, "partials fit a ring stage");
  float* const norm_part = reinterpret_cast<float*>(&ring[kLinearStages - 1][0]);

  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int c = lane % 16, g = lane / 16;
  const int64_t tiles = a.n / 16;
  const int64_t my_tiles = (tiles - blockIdx.x + gridDim.x - 1) / gridDim.x;
  const int64_t total = my_tiles * kPasses;  // passes of this workgroup
  const bool row_ok = c < a.rows;
  const bf16x8_t zero = __builtin_bit_cast(bf16x8_t, v4u{0u, 0u, 0u, 0u});

  // DMA source of row r = 2*wave + i of tile 0: lane l reads 16-byte slot
  // l ^ r of each 1 KiB piece, so slot S lands at S ^ r
  const unsigned char* src[kRowsPerWave];
#pragma unroll
  for (int i = 0; i < kRowsPerWave; ++i) {
    const int r = wave * kRowsPerWave + i;
    src[i] = reinterpret_cast<const unsigned char*>(a.w + r * a.k) + 16 * (lane ^ r);
  }
  const int64_t tile_bytes = 16 * a.k * (int64_t)sizeof(bf16_t);
  const int64_t set_bytes = a.n * a.k * (int64_t)sizeof(bf16_t);  // gate rows -> up rows
  // LDS address of this lane's operand slot of chunk j in ring stage 0
  uint32_t rd[kChunks];
#pragma unroll
  for (int j = 0; j < kChunks; ++j) {
    const int slot = wave * (kWaveK / 8) + 4 * j + g;
    rd[j] = lds_off(&ring[0][c * kRowBytes + 16 * (slot ^ c)]);
  }

  // pass q of the stream (tile blockIdx.x + (q / kPasses) * gridDim.x, pass
  // kPass = q % kPasses of it) into ring stage q % 4
  auto issue = [&](int64_t q, auto pass_tag) {
    constexpr int kPass = decltype(pass_tag)::value % kPasses;
    constexpr int kStage = decltype(pass_tag)::value % kLinearStages;
    constexpr int kSet = kSets == 2 ? (kPass & 1) : 0;
    constexpr int kKp = kSets == 2 ? kPass >> 1 : kPass;
    const int64_t t = blockIdx.x + (q / kPasses) * gridDim.x;
    const int64_t off = t * tile_bytes + kSet * set_bytes + kKp * kRowBytes;
#pragma unroll
    for (int i = 0; i < kRowsPerWave; ++i) {
      const int r = wave * kRowsPerWave + i;
#pragma unroll
      for (int pc = 0; pc < kPieces; ++pc) {
        lds_dma16<kCacheStream>(src[i] + off + pc * kWave * 16, &ring[kStage][r * kRowBytes + pc * kWave * 16]);
      }
    }
  };

  // this wave's x operands of the whole k (its eighth of every pass).  The
  // loop uses them from its first step, so the compiler waits for them (and
  // for every load issued before that wait) ahead of the loop.  A workgroup
  // of one two-pass tile issues them between passes 0 and 1 (that wait is
  // then the one for pass 0 anyway); a longer stream settles them first, so
  // the ring starts full after one L2 round trip instead of draining.
  bf16x8_t xa[kKPasses][kChunks];
  auto load_x = [&]() {
    const bf16_t* xp = a.x + (int64_t)(row_ok ? c : 0) * a.x_stride + wave * kWaveK + 8 * g;
#pragma unroll
    for (int kp = 0; kp < kKPasses; ++kp) {
#pragma unroll
      for (int j = 0; j < kChunks; ++j) xa[kp][j] = row_ok ? load_bf16x8(xp + kp * kPassK + 32 * j) : zero;
    }
  };
  if constexpr (kNorm != kLinearNoNorm) {
    // RMSNorm of the rows in the arithmetic of rms_norm_kernel (h = x + res
    // rounded to bf16, fp32 sum of squares, y = w * (h / sqrt(mean + eps))
    // rounded once; only the order of the sum of squares differs).  The
    // loads are unconditional (a row past `rows` reads row 0; its values are
    // zeroed at the end) and settled by one wait before the first passes'
    // DMA goes out: conditional loads and loads still pending behind the DMA
    // would each make the compiler wait for every load in flight.  The
    // arithmetic then overlaps the DMA.
    constexpr bool kRes = kNorm == kLinearNormRes;
    const int64_t kofs = wave * kWaveK + 8 * g;
    const int64_t row = row_ok ? c : 0;
    v4u hv[kKPasses][kChunks], nw[kKPasses][kChunks], rv[kRes ? kKPasses : 1][kChunks];
#pragma unroll
    for (int kp = 0; kp < kKPasses; ++kp) {
#pragma unroll
      for (int j = 0; j < kChunks; ++j) {
        const int64_t col = kofs + kp * kPassK + 32 * j;
        hv[kp][j] = *reinterpret_cast<const v4u*>(a.x + row * a.x_stride + col);
        nw[kp][j] = *reinterpret_cast<const v4u*>(a.norm_w + col);
        if constexpr (kRes) rv[kp][j] = *reinterpret_cast<const v4u*>(a.res + row * a.res_stride + col);
      }
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    issue(0, std::integral_constant<int, 0>{});
    issue(1, std::integral_constant<int, 1>{});
    if (total > 2) issue(2, std::integral_constant<int, 2>{});
    // The sum of squares in rms_norm_kernel's order at k = 2048 (256 threads,
    // one 16-byte vector each): an fma chain over the vector's 8 elements, an
    // xor butterfly over each 64 vectors, the four sums added in order.  The
    // norm is then bit-identical to nie_rms_norm's.
#pragma unroll
    for (int kp = 0; kp < kKPasses; ++kp) {
#pragma unroll
      for (int j = 0; j < kChunks; ++j) {
        if constexpr (kRes) {
          v4u sum;
#pragma unroll
          for (int w2 = 0; w2 < 4; ++w2) {
            sum[w2] = pack_bf16x2(vec_elt<bf16_t>(hv[kp][j], 2 * w2) + vec_elt<bf16_t>(rv[kp][j], 2 * w2),
                                  vec_elt<bf16_t>(hv[kp][j], 2 * w2 + 1) + vec_elt<bf16_t>(rv[kp][j], 2 * w2 + 1));
          }
          hv[kp][j] = sum;
        }
        float ssv = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float h = vec_elt<bf16_t>(hv[kp][j], e);
          ssv = fmaf(h, h, ssv);
        }
        // vector index of (row c, column kofs + kp*1024 + 32 j)
        const int v = (int)((kofs + kp * kPassK + 32 * j) / 8);
        asm volatile("s_nop 1\n\tds_write_b32 %0, %1" ::"v"(lds_off(&norm_part[c * kNormVecs + v])), "v"(ssv)
                     : "memory");
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    // wave w reduces rows 2w and 2w + 1: lane l takes vectors 64 q + l
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
      const int r = 2 * wave + rr;
      uint32_t addr[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) addr[q] = lds_off(&norm_part[r * kNormVecs + 64 * q + lane]);
      uint32_t pv[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) asm volatile("ds_read_b32 %0, %1" : "=v"(pv[q]) : "v"(addr[q]));
      asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(pv[0]), "+v"(pv[1]), "+v"(pv[2]), "+v"(pv[3]));
      float row_ss = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float t = __uint_as_float(pv[q]);
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) t += __shfl_xor(t, off);
        row_ss += t;
      }
      if (lane == 0) {
        asm volatile("s_nop 1\n\tds_write_b32 %0, %1" ::"v"(lds_off(&norm_ss[r])), "v"(row_ss) : "memory");
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    uint32_t total_bits;
    asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(total_bits) : "v"(lds_off(&norm_ss[c])));
    const float denom = sqrtf(__uint_as_float(total_bits) * (1.f / (float)(kKPasses * kPassK)) + a.eps);
    const bool write_sum = kRes && blockIdx.x == 0 && a.sum_out != nullptr && row_ok;
#pragma unroll
    for (int kp = 0; kp < kKPasses; ++kp) {
#pragma unroll
      for (int j = 0; j < kChunks; ++j) {
        if (write_sum) {
          *reinterpret_cast<v4u*>(a.sum_out + (int64_t)c * a.sum_stride + kofs + kp * kPassK + 32 * j) = hv[kp][j];
        }
        float y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) y[e] = vec_elt<bf16_t>(nw[kp][j], e) * (vec_elt<bf16_t>(hv[kp][j], e) / denom);
        v4u o;
#pragma unroll
        for (int w2 = 0; w2 < 4; ++w2) o[w2] = row_ok ? pack_bf16x2(y[2 * w2], y[2 * w2 + 1]) : 0u;
        xa[kp][j] = __builtin_bit_cast(bf16x8_t, o);
      }
    }
  } else if (total > 2) {
    load_x();
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    issue(0, std::integral_constant<int, 0>{});
    issue(1, std::integral_constant<int, 1>{});
    issue(2, std::integral_constant<int, 2>{});
  } else {
    issue(0, std::integral_constant<int, 0>{});
    load_x();
    issue(1, std::integral_constant<int, 1>{});
  }

  v4f acc[kSets];
#pragma unroll
  for (int s = 0; s < kSets; ++s) acc[s] = v4f{0.f, 0.f, 0.f, 0.f};

  for (int64_t q0 = 0; q0 < total; q0 += kTrip) {
    static_for<0, kTrip>([&](auto u_tag) {
      constexpr int kU = decltype(u_tag)::value;
      constexpr int kStage = kU % kLinearStages;
      constexpr int kPass = kU % kPasses;
      constexpr int kSet = kSets == 2 ? (kPass & 1) : 0;
      constexpr int kKp = kSets == 2 ? kPass >> 1 : kPass;
      const int64_t q = q0 + kU;
      if (q >= total) return;  // uniform: the last trip may end early, at a tile boundary
      // passes q+1 and q+2 (when they exist) may still be in flight
      const int64_t after = total - 1 - q;
      if (after >= 2) __builtin_amdgcn_s_waitcnt(waitcnt_vm(2 * kOps));
      else if (after == 1) __builtin_amdgcn_s_waitcnt(waitcnt_vm(kOps));
      else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
      // every wave has its rows of pass q, and is done with stage (q - 1) % 4.
      // A bare s_barrier: __syncthreads() would first wait for every DMA in
      // flight, the next passes' included.
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      if (q + kLinearStages - 1 < total) issue(q + kLinearStages - 1, std::integral_constant<int, kU + kLinearStages - 1>{});
      uint32_t addr[kChunks];
#pragma unroll
      for (int j = 0; j < kChunks; ++j) addr[j] = rd[j] + kStage * kLinearPassBytes;
      uint4 wv[kChunks];
      ring_read_k<kChunks>(wv, addr);
#pragma unroll
      for (int j = 0; j < kChunks; ++j) {
        acc[kSet] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[kKp][j], __builtin_bit_cast(bf16x8_t, wv[j]),
                                                            acc[kSet], 0, 0, 0);
      }
      if constexpr (kPass == kPasses - 1) {
        // the tile's sums meet in LDS; wave 0 writes them.  The next write of
        // red comes at least one pass (one barrier) later.  Inline-asm LDS
        // ops and an explicit lgkmcnt wait: compiler-visible LDS accesses
        // would first wait for the DMA still in flight.
        // The accumulators come straight from the MFMAs: a DS instruction
        // reading an MFMA result needs wait states after it (11 for the
        // 8-pass 16x16x32), which the compiler does not insert ahead of
        // inline asm, so the asm carries 16 of its own.
#pragma unroll
        for (int s = 0; s < kSets; ++s) {
          const v4u v = __builtin_bit_cast(v4u, acc[s]);
          asm volatile("s_nop 7\n\ts_nop 7\n\tds_write_b128 %0, %1" ::"v"(lds_off(&red[s][wave][lane])), "v"(v)
                       : "memory");
          acc[s] = v4f{0.f, 0.f, 0.f, 0.f};
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        if (wave == 0) {
          v4f sum[kSets];
#pragma unroll
          for (int s = 0; s < kSets; ++s) {
            uint32_t raddr[kLinearWaves];
#pragma unroll
            for (int w = 0; w < kLinearWaves; ++w) raddr[w] = lds_off(&red[s][w][lane]);
            uint4 part[kLinearWaves];
            ring_read_k<kLinearWaves>(part, raddr);
            sum[s] = __builtin_bit_cast(v4f, part[0]);
#pragma unroll
            for (int w = 1; w < kLinearWaves; ++w) sum[s] += __builtin_bit_cast(v4f, part[w]);
          }
          // lane l holds rows 4g..4g+3 of column col
          const int64_t col = (blockIdx.x + (q / kPasses) * gridDim.x) * 16 + c;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int m = 4 * g + r;
            if (m >= a.rows) break;
            float v;
            if constexpr (kEpi == kLinearSiluMul) {
              const float gate = round_to_bf16(sum[0][r]);
              const float up = round_to_bf16(sum[1][r]);
              v = round_to_bf16(gate / (1.f + expf(-gate))) * up;
            } else {
              v = sum[0][r];
            }
            reinterpret_cast<uint16_t*>(a.y)[m * a.y_stride + col] = (uint16_t)f32_to_bf16_bits(v);
          }
        }
      }
    });
  }
}

// Floats -> one 16-byte vector of T (round to nearest even for bf16).
template <typename T>
__device__ __forceinline__ v4u pack_vec(const float (&y)[16 / Elt<T>::kBytes]) {
  v4u o;
  if constexpr (Elt<T>::kIsBf16) {
#pragma unroll
    for (int w = 0; w < 4; ++w) o[w] = pack_bf16x2(y[2 * w], y[2 * w + 1]);
  } else {
#pragma unroll
    for (int w = 0; w < 4; ++w) o[w] = __float_as_uint(y[w]);
  }
  return o;
}

// RoPE of 16-byte vectors: lo holds dims i..i+E-1 of the first half of a
// head, hi the same dims of the second half, c / s the cos / sin table
// entries of dims i.. at the token's position.  The arithmetic is
// rope_kv_append_kernel's (every product and sum rounded to T on its own):
// lo' = lo*c - hi*s, hi' = hi*c + lo*s.
template <typename T>
__device__ __forceinline__ void rope_vec(v4u& lo, v4u& hi, const v4u& c, const v4u& s) {
  constexpr int kE = 16 / Elt<T>::kBytes;
  float nlo[kE], nhi[kE];
#pragma unroll
  for (int e = 0; e < kE; ++e) {
    const float x1 = vec_elt<T>(lo, e), x2 = vec_elt<T>(hi, e);
    const float cc = vec_elt<T>(c, e), ss = vec_elt<T>(s, e);
    nlo[e] = sub_t<T>(mul_t<T>(x1, cc), mul_t<T>(x2, ss));
    nhi[e] = add_t<T>(mul_t<T>(x2, cc), mul_t<T>(x1, ss));
  }
  lo = pack_vec<T>(nlo);
  hi = pack_vec<T>(nhi);
}

// Merges nsplit split partials of one output row, one wave.  Split s of the
// row has its unnormalised O row at po + s*po_stride and its (max, sum) pair
// at ml + s*ml_stride.  The lanes form kSplitsPerPass groups of D/4 lanes; a
// group reads one split's O row as float4s.  Splits go in batches of
// kPasses * kSplitsPerPass: every load of a batch (the O rows, and one
// (max, sum) pair per lane) is issued before any is used, and batches
// combine through a running maximum, so the usual merge (<= 32 splits at
// head_dim 64) costs one memory round trip.
// The sum of the nsplit split partials of one row (the two-pass rounding's
// partials are shares of the normalised output, so they merge by plain
// addition), in the same fixed order as merge_row, rounded once.
// Agent-scope (coherent across the XCDs' L2s) stores and loads of four
// floats, as two 64-bit halves: how one workgroup hands another its split
// shares inside a launch.
__device__ __forceinline__ void store_agent4(float* p, float x, float y, float z, float w) {
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), (uint64_t)__float_as_uint(x) | ((uint64_t)__float_as_uint(y) << 32),
                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p + 2),
                     (uint64_t)__float_as_uint(z) | ((uint64_t)__float_as_uint(w) << 32), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float4 load_agent4(const float* p) {
  const uint64_t lo = __hip_atomic_load(reinterpret_cast<const uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const uint64_t hi =
      __hip_atomic_load(reinterpret_cast<const uint64_t*>(p + 2), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float4(__uint_as_float((uint32_t)lo), __uint_as_float((uint32_t)(lo >> 32)),
                     __uint_as_float((uint32_t)hi), __uint_as_float((uint32_t)(hi >> 32)));
}

// kAgent: the partials were stored by other workgroups of the running
// launch (store_agent4), so they are read with agent-scope loads.
template <typename T, int D, bool kAgent = false>
__device__ __forceinline__ void sum_row(const float* po, int64_t po_stride, int nsplit, T* out) {
  constexpr int kLanesPerSplit = D / 4;
  constexpr int kSplitsPerPass = kWave / kLanesPerSplit;
  constexpr int kPasses = 8;
  constexpr int kBatch = kPasses * kSplitsPerPass;
  const int lane = lane_id();
  const int sub = lane / kLanesPerSplit;
  const int chunk = lane % kLanesPerSplit;
  po += 4 * chunk;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s0 = 0; s0 < nsplit; s0 += kBatch) {
    const int count = min(kBatch, nsplit - s0);
    float4 v[kPasses];
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int sp = p * kSplitsPerPass + sub;
      if constexpr (kAgent) {
        v[p] = sp < count ? load_agent4(po + (s0 + sp) * po_stride) : make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        v[p] = sp < count ? *reinterpret_cast<const float4*>(po + (s0 + sp) * po_stride)
                          : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      acc.x += v[p].x;
      acc.y += v[p].y;
      acc.z += v[p].z;
      acc.w += v[p].w;
    }
  }
#pragma unroll
  for (int off = kLanesPerSplit; off < kWave; off <<= 1) {
    acc.x += __shfl_xor(acc.x, off);
    acc.y += __shfl_xor(acc.y, off);
    acc.z += __shfl_xor(acc.z, off);
    acc.w += __shfl_xor(acc.w, off);
  }
  if (sub == 0) store4<T>(out + 4 * chunk, acc.x, acc.y, acc.z, acc.w);
}

// sum_row over up to kRows rows at once (row n's split s at po + n *
// row_stride + s * po_stride, its output at out + n * out_stride): every
// row's loads of a batch are issued before any is added, and each row is
// summed in sum_row's order (the same bits).
template <typename T, int D, bool kAgent, int kRows>
__device__ __forceinline__ void sum_rows(const float* po, int64_t row_stride, int64_t po_stride, int nsplit, int rows,
                                         T* out, int64_t out_stride) {
  constexpr int kLanesPerSplit = D / 4;
  constexpr int kSplitsPerPass = kWave / kLanesPerSplit;
  constexpr int kPasses = 8;
  constexpr int kBatch = kPasses * kSplitsPerPass;
  const int lane = lane_id();
  const int sub = lane / kLanesPerSplit;
  const int chunk = lane % kLanesPerSplit;
  po += 4 * chunk;
  float4 acc[kRows];
#pragma unroll
  for (int n = 0; n < kRows; ++n) acc[n] = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s0 = 0; s0 < nsplit; s0 += kBatch) {
    const int count = min(kBatch, nsplit - s0);
    float4 v[kRows][kPasses];
#pragma unroll
    for (int n = 0; n < kRows; ++n) {
#pragma unroll
      for (int p = 0; p < kPasses; ++p) {
        const int sp = p * kSplitsPerPass + sub;
        const float* src = po + n * row_stride + (s0 + sp) * po_stride;
        if (n < rows && sp < count) {
          if constexpr (kAgent) {
            v[n][p] = load_agent4(src);
          } else {
            v[n][p] = *reinterpret_cast<const float4*>(src);
          }
        } else {
          v[n][p] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
    }
#pragma unroll
    for (int n = 0; n < kRows; ++n) {
#pragma unroll
      for (int p = 0; p < kPasses; ++p) {
        acc[n].x += v[n][p].x;
        acc[n].y += v[n][p].y;
        acc[n].z += v[n][p].z;
        acc[n].w += v[n][p].w;
      }
    }
  }
#pragma unroll
  for (int n = 0; n < kRows; ++n) {
#pragma unroll
    for (int off = kLanesPerSplit; off < kWave; off <<= 1) {
      acc[n].x += __shfl_xor(acc[n].x, off);
      acc[n].y += __shfl_xor(acc[n].y, off);
      acc[n].z += __shfl_xor(acc[n].z, off);
      acc[n].w += __shfl_xor(acc[n].w, off);
    }
    if (sub == 0 && n < rows) store4<T>(out + n * out_stride + 4 * chunk, acc[n].x, acc[n].y, acc[n].z, acc[n].w);
  }
}

template <typename T, int D>
__device__ __forceinline__ void merge_row(const float* po, int64_t po_stride, const float* ml, int64_t ml_stride,
                                          int nsplit, T* out) {
  constexpr int kLanesPerSplit = D / 4;
  constexpr int kSplitsPerPass = kWave / kLanesPerSplit;
  constexpr int kPasses = 8;
  constexpr int kBatch = kPasses * kSplitsPerPass;
  static_assert(kBatch <= kWave, "one (max, sum) pair per lane");
  const int lane = lane_id();
  const int sub = lane / kLanesPerSplit;
  const int chunk = lane % kLanesPerSplit;
  po += 4 * chunk;
  float run_max = kNegInf;
  float denom = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s0 = 0; s0 < nsplit; s0 += kBatch) {
    const int count = min(kBatch, nsplit - s0);
    float4 v[kPasses];
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int sp = p * kSplitsPerPass + sub;
      v[p] = sp < count ? *reinterpret_cast<const float4*>(po + (s0 + sp) * po_stride)
                        : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    const float2 mls = lane < count ? *reinterpret_cast<const float2*>(ml + (s0 + lane) * ml_stride)
                                    : make_float2(kNegInf, 0.f);
    float bmax = mls.x;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) bmax = fmaxf(bmax, __shfl_xor(bmax, off));
    const float new_max = fmaxf(run_max, bmax);
    const float keep = run_max == kNegInf ? 0.f : exp2f((run_max - new_max) * kLog2e);
    const float w = mls.x == kNegInf ? 0.f : exp2f((mls.x - new_max) * kLog2e);
    float dsum = w * mls.y;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) dsum += __shfl_xor(dsum, off);
    denom = denom * keep + dsum;
    acc.x *= keep;
    acc.y *= keep;
    acc.z *= keep;
    acc.w *= keep;
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const float ws = __shfl(w, p * kSplitsPerPass + sub);
      acc.x += ws * v[p].x;
      acc.y += ws * v[p].y;
      acc.z += ws * v[p].z;
      acc.w += ws * v[p].w;
    }
    run_max = new_max;
  }
#pragma unroll
  for (int off = kLanesPerSplit; off < kWave; off <<= 1) {
    acc.x += __shfl_xor(acc.x, off);
    acc.y += __shfl_xor(acc.y, off);
    acc.z += __shfl_xor(acc.z, off);
    acc.w += __shfl_xor(acc.w, off);
  }
  if (sub == 0) {
    const float inv = 1.f / denom;
    store4<T>(out + 4 * chunk, acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
  }
}

// merge_row over up to kRows rows at once (row n's split s at po + n *
// row_stride + s * po_stride and ml + n * ml_row_stride + s * ml_stride,
// its output at out + n * out_stride), reading partials that other
// workgroups of the running launch stored with agent-scope stores: every
// row's loads of a batch are issued before any is used, and each row is
// merged in merge_row's order (the same bits).
template <typename T, int D, int kRows>
__device__ __forceinline__ void merge_rows_agent(const float* po, int64_t row_stride, int64_t po_stride, const float* ml,
                                                 int64_t ml_row_stride, int64_t ml_stride, int nsplit, int rows,
                                                 T* out, int64_t out_stride) {
  constexpr int kLanesPerSplit = D / 4;
  constexpr int kSplitsPerPass = kWave / kLanesPerSplit;
  constexpr int kPasses = 8;
  constexpr int kBatch = kPasses * kSplitsPerPass;
  static_assert(kBatch <= kWave, "one (max, sum) pair per lane");
  const int lane = lane_id();
  const int sub = lane / kLanesPerSplit;
  const int chunk = lane % kLanesPerSplit;
  po += 4 * chunk;
  float run_max[kRows], denom[kRows];
  float4 acc[kRows];
#pragma unroll
  for (int n = 0; n < kRows; ++n) {
    run_max[n] = kNegInf;
    denom[n] = 0.f;
    acc[n] = make_float4(0.f, 0.f, 0.f, 0.f);
  }
  for (int s0 = 0; s0 < nsplit; s0 += kBatch) {
    const int count = min(kBatch, nsplit - s0);
    float4 v[kRows][kPasses];
    float2 mls[kRows];
#pragma unroll
    for (int n = 0; n < kRows; ++n) {
#pragma unroll
      for (int p = 0; p < kPasses; ++p) {
        const int sp = p * kSplitsPerPass + sub;
        v[n][p] = (n < rows && sp < count) ? load_agent4(po + n * row_stride + (s0 + sp) * po_stride)
                                           : make_float4(0.f, 0.f, 0.f, 0.f);
      }
      if (n < rows && lane < count) {
        const uint64_t bits = __hip_atomic_load(
            reinterpret_cast<const uint64_t*>(ml + n * ml_row_stride + (s0 + lane) * ml_stride), __ATOMIC_RELAXED,
            __HIP_MEMORY_SCOPE_AGENT);
        mls[n] = make_float2(__uint_as_float((uint32_t)bits), __uint_as_float((uint32_t)(bits >> 32)));
      } else {
        mls[n] = make_float2(kNegInf, 0.f);
      }
    }
#pragma unroll
    for (int n = 0; n < kRows; ++n) {
      float bmax = mls[n].x;
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) bmax = fmaxf(bmax, __shfl_xor(bmax, off));
      const float new_max = fmaxf(run_max[n], bmax);
      const float keep = run_max[n] == kNegInf ? 0.f : exp2f((run_max[n] - new_max) * kLog2e);
      const float w = mls[n].x == kNegInf ? 0.f : exp2f((mls[n].x - new_max) * kLog2e);
      float dsum = w * mls[n].y;
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) dsum += __shfl_xor(dsum, off);
      denom[n] = denom[n] * keep + dsum;
      acc[n].x *= keep;
      acc[n].y *= keep;
      acc[n].z *= keep;
      acc[n].w *= keep;
#pragma unroll
      for (int p = 0; p < kPasses; ++p) {
        const float ws = __shfl(w, p * kSplitsPerPass + sub);
        acc[n].x += ws * v[n][p].x;
        acc[n].y += ws * v[n][p].y;
        acc[n].z += ws * v[n][p].z;
        acc[n].w += ws * v[n][p].w;
      }
      run_max[n] = new_max;
    }
  }
#pragma unroll
  for (int n = 0; n < kRows; ++n) {
#pragma unroll
    for (int off = kLanesPerSplit; off < kWave; off <<= 1) {
      acc[n].x += __shfl_xor(acc[n].x, off);
      acc[n].y += __shfl_xor(acc[n].y, off);
      acc[n].z += __shfl_xor(acc[n].z, off);
      acc[n].w += __shfl_xor(acc[n].w, off);
    }
    if (sub == 0 && n < rows) {
      const float inv = 1.f / denom[n];
      store4<T>(out + n * out_stride + 4 * chunk, acc[n].x * inv, acc[n].y * inv, acc[n].z * inv, acc[n].w * inv);
    }
  }
}

// Heads per decode workgroup: as many as fill a 1 KiB row slice, capped by
// the largest power of two dividing kv_heads (so every wave has a head).
template <typename T, int D>
constexpr int decode_max_heads() {
  return (kWave * 16) / (D * Elt<T>::kBytes) > kDecodeWaves ? kDecodeWaves : (kWave * 16) / (D * Elt<T>::kBytes);
}

constexpr int kDecodeLdsBudget = 160 * 1024;


template <typename T, int D, int kHeads>
constexpr int decode_stages() {
  constexpr int per_stage = 2 * GroupTile<T, D, kHeads>::kBytes;
  return kDecodeLdsBudget / per_stage >= 4 ? 4 : (kDecodeLdsBudget / per_stage >= 3 ? 3 : 2);
}

// One workgroup = one (sequence, key split, head group); wave w handles KV
// head group*kHeads + w and its GQA query heads.  kMergeLast: the build for
// calls whose splits merge inside the kernel (DecodeArgs::merge_last); its
// merge needs more VGPRs than the loop, so the other calls run a build
// without it.
template <typename T, int D, bool kUniform, int kHeads, bool kMergeLast = false>
__global__ __launch_bounds__(kHeads* kWave) void paged_decode_kernel(DecodeArgs a, DecodeItems items) {
  using F = Frag<T, D>;
  using GT = GroupTile<T, D, kHeads>;
  constexpr int kStages = decode_stages<T, D, kHeads>();
  constexpr int kStageBytes = 2 * GT::kBytes;  // K tile then V tile
  constexpr int kOwnOps = 2 * GT::kOpsPerWave;  // DMA ops one wave issues per tile
  constexpr int kEltPerChunk = 16 / Elt<T>::kBytes;
  __shared__ __attribute__((aligned(16))) unsigned char ring[kStages][kStageBytes];

  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int g = lane >> 4;
  const int row = lane & 15;

  int64_t b, split, first_item, nsplit, tps;
  int seq_len;
  if (a.dev_items != nullptr && a.dev_items->count > 0) {
    // the host's plan of this step, in device memory (scalar loads)
    const DecodeItems* __restrict__ d = a.dev_items;
    if ((int)blockIdx.x >= d->count) return;  // uniform over the workgroup
    const uint32_t it = d->item[blockIdx.x];
    b = it >> 16;
    split = it & 0xffffu;
    seq_len = d->seq_len[b];
    first_item = d->seq_first[b];
    tps = d->tps;
    nsplit = cdiv(cdiv((int64_t)seq_len, (int64_t)kTileKeys), tps);
  } else if (items.count > 0) {
    if ((int)blockIdx.x >= items.count) return;  // uniform over the workgroup
    const uint32_t it = items.item[blockIdx.x];
    b = it >> 16;
    split = it & 0xffffu;
    seq_len = items.seq_len[b];
    first_item = items.seq_first[b];
    tps = a.tiles_per_split;
    nsplit = cdiv(cdiv((int64_t)seq_len, (int64_t)kTileKeys), tps);
  } else {
    // the lengths are read once: the split length (planned on the device
    // when the host sent none) and the item's sequence come out of them
    int first_len;
    tps = decode_call_tps(a, &first_len);
    locate_item((int64_t)blockIdx.x, a.batch, [&](int64_t s) { return decode_splits_of(a, s, tps, first_len); },
                &b, &split, &first_item, &nsplit);
    if (b < 0) return;  // uniform over the workgroup
    // lane b already holds the length of one of the first 64 sequences
    seq_len = b < kWave ? __shfl(first_len, (int)b) : a.seq_lens[b];
  }
  seq_len = __builtin_amdgcn_readfirstlane(seq_len);
  const int tiles_per_split = (int)tps;
  const int h0 = (int)blockIdx.y * kHeads;  // first KV head of the group
  const int h = h0 + wave;

  const int32_t* table = a.tables + b * a.table_stride;
  const int tlen = (int)a.table_stride;
  const int key_begin = (int)split * tiles_per_split * kTileKeys;
  const int key_end = min(key_begin + tiles_per_split * kTileKeys, seq_len);
  const int last = key_end - 1;

  const T* kc = reinterpret_cast<const T*>(a.k_cache) + h0 * D;
  const T* vc = reinterpret_cast<const T*>(a.v_cache) + h0 * D;

  // Q^T operand: row -> query head h*group + row (rows >= group are zero).
  F qf;
  const bool row_valid = row < a.group;
  const int qh = h * a.group + row;
  if (row_valid) {
    load_slice<T, D>(qf, reinterpret_cast<const T*>(a.q) + b * a.q_sb + qh * a.q_sh);
  } else {
#pragma unroll
    for (int i = 0; i < F::kVec; ++i) qf.v[i] = uint4{0u, 0u, 0u, 0u};
  }

  SoftmaxState<D> st;
  st.init();

  // Fused append: the workgroup whose split ends the sequence takes the new
  // K/V row of position seq_len - 1.  In wave w, lanes [0, kHeadChunks)
  // carry the 16-byte K chunks of head h0 + w and the next kHeadChunks lanes
  // its V chunks.  At the last tile the wave writes them over its LDS copy of
  // that row (only this wave reads its head's chunks), and once the ring has
  // drained, into the cache slot of the position.  A table entry outside the
  // pool skips both, as an out-of-range slot skips nie_kv_append.
  constexpr int kHeadChunks = D * Elt<T>::kBytes / 16;
  const bool appender = a.k_new != nullptr && key_end == seq_len;  // uniform over the workgroup
  const bool carrier = appender && lane < 2 * kHeadChunks;
  const bool carries_k = lane < kHeadChunks;
  const int new_c = carries_k ? lane : lane - kHeadChunks;  // chunk within the head's row
  v4u new_chunk;  // defined on carrier lanes, used only there
  if (carrier) {
    const T* src = reinterpret_cast<const T*>(carries_k ? a.k_new : a.v_new) + b * (carries_k ? a.kn_s : a.vn_s) +
                   h * D + new_c * kEltPerChunk;
    new_chunk = *reinterpret_cast<const v4u*>(src);
  }
  bool carry = false;  // set at the last tile: the chunk goes to new_dst
  T* new_dst = nullptr;
  // RoPE (with the fused append): this lane's cos / sin vectors for the
  // first-half dims of its q vectors, and for its new K chunk's dims
  const bool rope = a.rope_cos != nullptr && a.k_new != nullptr;
  constexpr int kQHalf = F::kVec / 2;
  v4u q_cos[kQHalf], q_sin[kQHalf], k_cos = v4u{0u, 0u, 0u, 0u}, k_sin = v4u{0u, 0u, 0u, 0u};
  if (rope) {
    int64_t pos = seq_len - 1;
    pos = pos >= a.rope_rows ? a.rope_rows - 1 : pos;
    const T* crow = reinterpret_cast<const T*>(a.rope_cos) + pos * (D / 2);
    const T* srow = reinterpret_cast<const T*>(a.rope_sin) + pos * (D / 2);
#pragma unroll
    for (int j = 0; j < kQHalf; ++j) {
      const int d0 = (64 * j + 16 * (lane >> 4)) / Elt<T>::kBytes;  // first dim of q vector j
      q_cos[j] = *reinterpret_cast<const v4u*>(crow + d0);
      q_sin[j] = *reinterpret_cast<const v4u*>(srow + d0);
    }
    if (carrier && carries_k) {
      const int d0 = (new_c % (kHeadChunks / 2)) * kEltPerChunk;
      k_cos = *reinterpret_cast<const v4u*>(crow + d0);
      k_sin = *reinterpret_cast<const v4u*>(srow + d0);
    }
  }

  TableCache tc;
  if constexpr (kUniform) tc.load(table, tlen, key_begin >> a.geom.bs_shift);
  // the new chunk's load completes with the table loads (one round trip)
  asm volatile("" : "+v"(new_chunk));

  // This wave's share of the DMA ops of a tile: op = wave + i*kHeads; in op
  // `op`, lane l fills LDS position op*64 + l, i.e. row r = op*kRowsPerOp +
  // l/kChunks, chunk position l%kChunks, which holds global chunk
  // position ^ swz(r).  Keys past the end of the split are clamped to its
  // last key (so no lane reads a slot the sequence does not own; those keys
  // are masked to p = 0).
  auto issue = [&](int slot, int key0) {
    TileAddr<kUniform, false> ta;  // a split covers <= kTableWindow tiles, so <= kTableWindow blocks
    ta.init(a.geom, table, tlen, tc, key0);
    const int lim = last - key0;
    unsigned char* kdst = &ring[slot][0];
    unsigned char* vdst = kdst + GT::kBytes;
#pragma unroll
    for (int i = 0; i < GT::kOpsPerWave; ++i) {
      const int op = wave + i * kHeads;
      const int r = op * GT::kRowsPerOp + lane / GT::kChunks;
      const int chunk = (lane % GT::kChunks) ^ GT::swz(r);
      const int64_t src = ta.at(a.geom, table, tlen, key0, min(r, lim)) + chunk * kEltPerChunk;
      lds_dma16<kCacheStream>(kc + src, kdst + op * kWave * 16);
      lds_dma16<kCacheStream>(vc + src, vdst + op * kWave * 16);
    }
  };

  // Per-lane LDS offsets inside a stage (tile independent): the K slice
  // chunks and the sixteen V^T elements of the bf16 path.
  uint32_t koff[F::kVec];
#pragma unroll
  for (int j = 0; j < F::kVec; ++j) {
    koff[j] = GT::chunk_offset(row, (wave * D * Elt<T>::kBytes + 64 * j + 16 * g) >> 4);
  }
  uint32_t voff[(D / 16) * 4];  // fp32: V^T elements read one by one
  uint32_t vtr[D / 16];         // bf16: transposing reads
#pragma unroll
  for (int c = 0; c < D / 16; ++c) {
    vtr[c] = GT::kBytes + GT::vt_offset(lane, wave, c);
#pragma unroll
    for (int e = 0; e < 4; ++e) voff[4 * c + e] = GT::kBytes + GT::elt_offset(4 * g + e, wave, 16 * c + row);
  }

  auto consume = [&](int slot, int key0) {
    const unsigned char* stage = &ring[slot][0];
    F kf;
    if constexpr (Elt<T>::kIsBf16) {
      const uint32_t base = lds_off(stage);
      uint32_t ka[F::kVec];
#pragma unroll
      for (int j = 0; j < F::kVec; ++j) ka[j] = base + koff[j];
      ring_read_k<F::kVec>(kf.v, ka);
    } else {
#pragma unroll
      for (int j = 0; j < F::kVec; ++j) kf.v[j] = *reinterpret_cast<const uint4*>(stage + koff[j]);
    }
    v4f s = qk_mfma<T, D>(kf, qf);
#pragma unroll
    for (int i = 0; i < 4; ++i) s[i] = scaled_score<T>(s[i], a.scale);
    if (key0 + kTileKeys - 1 > last) {  // only the split's last tile can pass its end
#pragma unroll
      for (int i = 0; i < 4; ++i) s[i] = (key0 + 4 * g + i <= last) ? s[i] : kNegInf;
    }
    softmax_tile<D>(st, s);
    if constexpr (Elt<T>::kIsBf16) {
      const v4s pb = pack_bf16x4(s[0], s[1], s[2], s[3]);
      const uint32_t base = lds_off(stage);
#pragma unroll
      for (int c0 = 0; c0 < D / 16; c0 += 4) {
        uint32_t va[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) va[i] = base + vtr[c0 + i];
        v4s vt[4];
        ring_read_vt4(vt, va);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          st.o[c0 + c] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vt[c], pb, st.o[c0 + c], 0, 0, 0);
        }
      }
    } else {
#pragma unroll
      for (int c = 0; c < D / 16; ++c) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float v = *reinterpret_cast<const float*>(stage + voff[4 * c + j]);
          st.o[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(v, s[j], st.o[c], 0, 0, 0);
        }
      }
    }
  };

  const int ntiles = (key_end - key_begin + kTileKeys - 1) / kTileKeys;
  constexpr int kAhead = kStages - 1;
  // only tiles the split has are fetched: a tail shorter than the ring
  // leaves stages unused instead of re-reading its last tile
#pragma unroll
  for (int j = 0; j < kAhead; ++j) {
    if (j < ntiles) issue(j, key_begin + j * kTileKeys);
  }
  if (rope) {
    // rotate q (vector j pairs with vector j + kVec/2: dims i and i + D/2)
    // while the first tiles are in flight
    if (row_valid) {
#pragma unroll
      for (int j = 0; j < kQHalf; ++j) {
        v4u lo = __builtin_bit_cast(v4u, qf.v[j]), hi = __builtin_bit_cast(v4u, qf.v[j + kQHalf]);
        rope_vec<T>(lo, hi, q_cos[j], q_sin[j]);
        qf.v[j] = __builtin_bit_cast(uint4, lo);
        qf.v[j + kQHalf] = __builtin_bit_cast(uint4, hi);
      }
    }
    if (appender) {
      // K chunk c pairs with chunk c + kHeadChunks/2 (lane xor kHeadChunks/2)
      v4u other;
#pragma unroll
      for (int w = 0; w < 4; ++w) other[w] = (uint32_t)__shfl_xor((int)new_chunk[w], kHeadChunks / 2);
      if (carrier && carries_k) {
        const bool first_half = new_c < kHeadChunks / 2;
        v4u lo = first_half ? new_chunk : other, hi = first_half ? other : new_chunk;
        rope_vec<T>(lo, hi, k_cos, k_sin);
        new_chunk = first_half ? lo : hi;
      }
    }
  }
  for (int t = 0; t < ntiles; t += kStages) {
#pragma unroll
    for (int j = 0; j < kStages; ++j) {
      const int tt = t + j;
      if (tt >= ntiles) break;  // uniform over the workgroup
      // this wave's ops for tile tt are done once at most the ops of the
      // tiles issued after it (min(kAhead - 1, ntiles - 1 - tt) of them) are
      // outstanding; the barrier extends that to every wave and guarantees
      // that every wave has finished reading tile tt-1, whose stage the next
      // fetch reuses
      wait_dma_groups<kOwnOps, kAhead - 1>(min(kAhead - 1, ntiles - 1 - tt));
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      if (tt + kAhead < ntiles) issue((j + kAhead) % kStages, key_begin + (tt + kAhead) * kTileKeys);
      __builtin_amdgcn_sched_barrier(0);
      if (appender && tt == ntiles - 1) {
        const int pos = seq_len - 1;
        int lb, off;
        if (a.geom.bs_shift >= 0) {
          lb = pos >> a.geom.bs_shift;
          off = pos & (a.geom.block_size - 1);
        } else {
          lb = (int)((uint32_t)pos / (uint32_t)a.geom.block_size);
          off = pos - lb * a.geom.block_size;
        }
        int phys;
        if constexpr (kUniform) {
          phys = tc.template lookup<false>(table, tlen, lb);  // the split's blocks are in the window
        } else {
          phys = table[lb];
        }
        if (carrier && lb < tlen && phys >= 0 && phys < a.geom.num_blocks) {
          T* cache = reinterpret_cast<T*>(const_cast<void*>(carries_k ? a.k_cache : a.v_cache));
          new_dst = cache + a.geom.layer_offset + ((int64_t)phys * a.geom.block_size + off) * a.geom.row_elems +
                    h * D + new_c * kEltPerChunk;
          carry = true;
          // The rows after the new token's were read from its slot too (reads
          // past the split's last key clamp to it; those keys are masked,
          // but their V rows still meet p = 0 in the P.V MFMAs, so they must
          // hold the new row, not the slot's old content).  The wait +
          // barrier above ordered the tile's DMA before these writes.
          const uint32_t base = lds_off(&ring[j][0]) + (carries_k ? 0u : (uint32_t)GT::kBytes);
          for (int rr = pos - key_begin - tt * kTileKeys; rr < kTileKeys; ++rr) {
            const uint32_t patch = base + (uint32_t)GT::chunk_offset(rr, wave * kHeadChunks + new_c);
            asm volatile("ds_write_b128 %0, %1" : : "v"(patch), "v"(new_chunk) : "memory");
          }
          asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      consume(j, key_begin + tt * kTileKeys);
    }
  }

  // every fetch has been waited for (the last tile's wait is vmcnt(0))
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  if (carry) *reinterpret_cast<v4u*>(new_dst) = new_chunk;
  const float lsum = sum_over_groups(st.lsum);
  if (nsplit == 1) {
    if (!row_valid) return;
    const float inv = 1.f / lsum;
    T* dst = reinterpret_cast<T*>(a.out) + b * a.o_sb + qh * a.o_sh + 4 * g;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      store4<T>(dst + 16 * c, st.o[c][0] * inv, st.o[c][1] * inv, st.o[c][2] * inv,
                st.o[c][3] * inv);
    }
    return;
  }
  // Split-K: store this split's partial (unnormalised O, running max, sum)
  // for the merge.  The bound keeps inconsistent length hints from writing
  // outside the workspace.
  const int64_t item = first_item + split;
  if constexpr (kMergeLast) {
    // Through to memory (agent scope), then counted on the (sequence, KV
    // head) counter; the wave that counts the last split merges every
    // split's partial of its query heads, in decode_merge_kernel's order,
    // and starts the counter over.  The bound holds for all splits of a
    // sequence or for none, so either every split counts or none does.
    if (a.ws_o == nullptr || first_item + nsplit > a.ws_items) return;
    if (row_valid) {
      float* dst = a.ws_o + (item * a.q_heads + qh) * D + 4 * g;
#pragma unroll
      for (int c = 0; c < D / 16; ++c) store_agent4(dst + 16 * c, st.o[c][0], st.o[c][1], st.o[c][2], st.o[c][3]);
      if (g == 0) {
        __hip_atomic_store(reinterpret_cast<uint64_t*>(a.ws_ml + (item * a.q_heads + qh) * 2),
                           (uint64_t)__float_as_uint(st.m) | ((uint64_t)__float_as_uint(lsum) << 32),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
    const int64_t pair = b * a.geom.kv_heads + h;
    uint32_t before = 0;
    if (lane == 0) {
      before = __hip_atomic_fetch_add(&a.ctl->pair[pair].done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    before = __builtin_amdgcn_readfirstlane(before);
    if (before != (uint32_t)nsplit - 1u) return;
    const int qh0 = h * a.group;
    for (int r0 = 0; r0 < a.group; r0 += 2) {
      merge_rows_agent<T, D, 2>(a.ws_o + (first_item * a.q_heads + qh0 + r0) * D, D, (int64_t)a.q_heads * D,
                                a.ws_ml + (first_item * a.q_heads + qh0 + r0) * 2, 2, (int64_t)a.q_heads * 2,
                                (int)nsplit, min(2, a.group - r0),
                                reinterpret_cast<T*>(a.out) + b * a.o_sb + (qh0 + r0) * a.o_sh, a.o_sh);
    }
    if (lane == 0) __hip_atomic_store(&a.ctl->pair[pair].done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  if (!row_valid || a.ws_o == nullptr || item >= a.ws_items) return;
  float* dst = a.ws_o + (item * a.q_heads + qh) * D + 4 * g;
#pragma unroll
  for (int c = 0; c < D / 16; ++c) {
    *reinterpret_cast<float4*>(dst + 16 * c) = make_float4(st.o[c][0], st.o[c][1], st.o[c][2], st.o[c][3]);
  }
  if (g == 0) *reinterpret_cast<float2*>(a.ws_ml + (item * a.q_heads + qh) * 2) = make_float2(st.m, lsum);
}

// ---------------------------------------------------------------------------
// Decode with the reference's rounding point.  paged_decode_kernel rounds
// exp(s - running max) to bf16 and divides O by the row sum at the end; the
// reference rounds the normalised probabilities exp(s - m) / l to bf16
// before P.V (layers/paged_attention.py:109-114), which needs each row's
// final (m, l) before any probability is formed.  Two passes over the keys,
// each a launch of decode_pass_kernel over the same work items:
//   kDecodeScores reads K, writes every key's score bf16(bf16(q.k) * scale)
//     (the reference's softmax input) to the workspace, and each split's
//     (max, sum of e^(s - max)) (v_exp_f32 exponentials, a step's summed in
//     fp32 and the steps in fp64: the sum's relative error stays near
//     2^-24, which moves the bf16 rounding of P = e / l for about one
//     probability in 10^4-10^5);
//   kDecodePV reads V and the scores, combines its row's (m, l) over all the
//     sequence's splits, and accumulates bf16(e^(s - m) / l) . V in fp32:
//     its share of the normalised output, which decode_merge_kernel<kSum>
//     adds up over the splits (or, with one split, it rounds and stores).
// Each pass reads one of K and V, half the bytes of the fused kernel per
// key, so a loop iteration covers two 16-key tiles (32 keys): one barrier
// and one dependent chain (LDS read, MFMA, softmax arithmetic) per 32 KiB
// of a workgroup's heads instead of per 16 KiB, with v_mfma_f32_16x16x32_bf16
// joining the two tiles (K slot 8(l/16) + e is key 4(l/16) + e of the first
// tile for e < 4 and of the second otherwise, on both operands).  The
// scores pass also does the fused append (and RoPE): the new K row patches
// its LDS copy, and the new K and V rows go to the cache, which the P.V
// pass then reads.
// Score layout: item i, KV head h, tile t, query row n (of the group),
// key k at (((i * kv_heads + h) * tps + t) * group + n) * 16 + k, bf16.
// ---------------------------------------------------------------------------
constexpr int kDecodeScores = 1;
constexpr int kDecodePV = 2;
constexpr int kPassStepTiles = 2;  // 16-key tiles per loop iteration

template <typename T, int D, int kHeads, int kPass>
constexpr int decode_pass_stage_bytes() {
  constexpr int tiles = kPassStepTiles * GroupTile<T, D, kHeads>::kBytes;
  // the P.V pass adds 1 KiB of scores per wave (one DMA op: the head's
  // group x 32 keys, at most 1 KiB)
  return kPass == kDecodeScores ? tiles : tiles + kHeads * kWave * 16;
}

template <typename T, int D, int kHeads, int kPass>
constexpr int decode_pass_stages() {
  constexpr int fit = kDecodeLdsBudget / decode_pass_stage_bytes<T, D, kHeads, kPass>();
  return fit >= 4 ? 4 : (fit >= 2 ? fit : 2);
}

// The work item of a decode workgroup (blockIdx.x): from the plan in device
// memory, from the kernel arguments, or located on the device from the
// lengths; false past the call's items (uniform over the workgroup).
struct DecodeWork {
  int64_t b, split, first_item, nsplit, tps;
  int seq_len;
};

__device__ __forceinline__ bool decode_work(const DecodeArgs& a, const DecodeItems& items, DecodeWork& w) {
  if (a.dev_items != nullptr && a.dev_items->count > 0) {
    const DecodeItems* __restrict__ d = a.dev_items;
    if ((int)blockIdx.x >= d->count) return false;
    const uint32_t it = d->item[blockIdx.x];
    w.b = it >> 16;
    w.split = it & 0xffffu;
    w.seq_len = d->seq_len[w.b];
    w.first_item = d->seq_first[w.b];
    w.tps = d->tps;
  } else if (items.count > 0) {
    if ((int)blockIdx.x >= items.count) return false;
    const uint32_t it = items.item[blockIdx.x];
    w.b = it >> 16;
    w.split = it & 0xffffu;
    w.seq_len = items.seq_len[w.b];
    w.first_item = items.seq_first[w.b];
    w.tps = a.tiles_per_split;
  } else {
    int first_len;
    w.tps = decode_call_tps(a, &first_len);
    int64_t count;
    const int64_t tps = w.tps;
    locate_item((int64_t)blockIdx.x, a.batch, [&](int64_t s) { return decode_splits_of(a, s, tps, first_len); },
                &w.b, &w.split, &w.first_item, &count);
    if (w.b < 0) return false;
    w.seq_len = w.b < kWave ? __shfl(first_len, (int)w.b) : a.seq_lens[w.b];
  }
  w.seq_len = __builtin_amdgcn_readfirstlane(w.seq_len);
  w.nsplit = cdiv(cdiv((int64_t)w.seq_len, (int64_t)kTileKeys), w.tps);
  return true;
}

template <typename T, int D, bool kUniform, int kHeads, int kPass>
__global__ __launch_bounds__(kHeads* kWave) void decode_pass_kernel(DecodeArgs a, DecodeItems items) {
  static_assert(Elt<T>::kIsBf16, "the reference rounding point matters for bf16 probabilities");
  static_assert(kPass == kDecodeScores || kPass == kDecodePV, "a pass of the two-pass decode");
  using F = Frag<T, D>;
  using GT = GroupTile<T, D, kHeads>;
  constexpr int kStages = decode_pass_stages<T, D, kHeads, kPass>();
  constexpr int kStageBytes = decode_pass_stage_bytes<T, D, kHeads, kPass>();
  constexpr int kTilesBytes = kPassStepTiles * GT::kBytes;
  constexpr int kOwnOps = kPassStepTiles * GT::kOpsPerWave + (kPass == kDecodePV ? 1 : 0);
  constexpr int kEltPerChunk = 16 / Elt<T>::kBytes;
  constexpr int kStepKeys = kPassStepTiles * kTileKeys;
  __shared__ __attribute__((aligned(16))) unsigned char ring[kStages][kStageBytes];

  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int g = lane >> 4;
  const int row = lane & 15;

  DecodeWork w;
  if (!decode_work(a, items, w)) return;
  const int64_t b = w.b;
  const int64_t nsplit = w.nsplit;
  const int64_t item = w.first_item + w.split;
  const int seq_len = w.seq_len;
  const int tps = (int)w.tps;
  const int h0 = (int)blockIdx.y * kHeads;
  const int h = h0 + wave;
  const int group = a.group;
  const int32_t* table = a.tables + b * a.table_stride;
  const int tlen = (int)a.table_stride;
  const int key_begin = (int)w.split * tps * kTileKeys;
  const int key_end = min(key_begin + tps * kTileKeys, seq_len);
  const int last = key_end - 1;
  const int ntiles = (key_end - key_begin + kTileKeys - 1) / kTileKeys;
  const int last_key0 = key_begin + (ntiles - 1) * kTileKeys;  // first key of the split's last tile
  const int nsteps = (ntiles + kPassStepTiles - 1) / kPassStepTiles;
  const bool row_valid = row < group;
  const int qh = h * group + row;

  // this item's scores and the sequence's (max, sum) pairs lie inside the
  // workspace (uniform); otherwise (lengths inconsistent with the host's
  // bounds) no score is written and the P.V pass does nothing
  const bool ws_ok = a.ws_s != nullptr && (item + 1) * tps * kTileKeys <= a.ws_s_keys && a.ws_ml != nullptr &&
                     w.first_item + nsplit <= a.ws_items;
  if constexpr (kPass == kDecodePV) {
    if (!ws_ok) return;
  }
  // the head's score rows of this item: tile t, row n, key k at (t * group + n) * 16 + k
  uint16_t* const hscores = ws_ok ? a.ws_s + ((item * a.geom.kv_heads + h) * tps) * group * kTileKeys : nullptr;

  // P.V pass: the (max, sum) pairs of every split of the sequence, loaded in
  // batches (lane group g takes splits g, g + 4, ...) before anything waits
  // for them; they are combined once the first tiles are on their way
  constexpr int kMlBatch = 8;
  float2 ml_first[kMlBatch];
  if constexpr (kPass == kDecodePV) {
#pragma unroll
    for (int j = 0; j < kMlBatch; ++j) {
      const int64_t sp = 4 * j + g;
      ml_first[j] = (row_valid && sp < nsplit)
                        ? *reinterpret_cast<const float2*>(a.ws_ml + ((w.first_item + sp) * a.q_heads + qh) * 2)
                        : make_float2(kNegInf, 0.f);
    }
  }

  // scores pass: q (rows >= group are zero)
  F qf;
  if (kPass == kDecodeScores && row_valid) {
    load_slice<T, D>(qf, reinterpret_cast<const T*>(a.q) + b * a.q_sb + qh * a.q_sh);
  } else {
#pragma unroll
    for (int i = 0; i < F::kVec; ++i) qf.v[i] = uint4{0u, 0u, 0u, 0u};
  }

  // Fused append (scores pass, the split that ends the sequence): lanes
  // [0, kHeadChunks) of wave w carry the 16-byte K chunks of head h0 + w,
  // the next kHeadChunks lanes its V chunks (as in paged_decode_kernel).
  constexpr int kHeadChunks = D * Elt<T>::kBytes / 16;
  const bool appender = kPass == kDecodeScores && a.k_new != nullptr && key_end == seq_len;
  const bool carrier = appender && lane < 2 * kHeadChunks;
  const bool carries_k = lane < kHeadChunks;
  const int new_c = carries_k ? lane : lane - kHeadChunks;
  v4u new_chunk = v4u{0u, 0u, 0u, 0u};
  if (carrier) {
    const T* src = reinterpret_cast<const T*>(carries_k ? a.k_new : a.v_new) + b * (carries_k ? a.kn_s : a.vn_s) +
                   h * D + new_c * kEltPerChunk;
    new_chunk = *reinterpret_cast<const v4u*>(src);
  }
  const bool rope = appender && a.rope_cos != nullptr;
  constexpr int kQHalf = F::kVec / 2;
  v4u q_cos[kQHalf], q_sin[kQHalf], k_cos = v4u{0u, 0u, 0u, 0u}, k_sin = v4u{0u, 0u, 0u, 0u};
  if (kPass == kDecodeScores && a.rope_cos != nullptr && a.k_new != nullptr) {
    int64_t pos = seq_len - 1;
    pos = pos >= a.rope_rows ? a.rope_rows - 1 : pos;
    const T* crow = reinterpret_cast<const T*>(a.rope_cos) + pos * (D / 2);
    const T* srow = reinterpret_cast<const T*>(a.rope_sin) + pos * (D / 2);
#pragma unroll
    for (int j = 0; j < kQHalf; ++j) {
      const int d0 = (64 * j + 16 * (lane >> 4)) / Elt<T>::kBytes;
      q_cos[j] = *reinterpret_cast<const v4u*>(crow + d0);
      q_sin[j] = *reinterpret_cast<const v4u*>(srow + d0);
    }
    if (carrier && carries_k) {
      const int d0 = (new_c % (kHeadChunks / 2)) * kEltPerChunk;
      k_cos = *reinterpret_cast<const v4u*>(crow + d0);
      k_sin = *reinterpret_cast<const v4u*>(srow + d0);
    }
  }

  TableCache tc;
  if constexpr (kUniform) tc.load(table, tlen, key_begin >> a.geom.bs_shift);
  asm volatile("" : "+v"(new_chunk));

  const T* src_cache = reinterpret_cast<const T*>(kPass == kDecodeScores ? a.k_cache : a.v_cache) + h0 * D;
  // P.V pass: the wave's score op per step reads the head's group x 16
  // scores of the step's tiles (2 x group 16-byte chunks per tile; lanes
  // past them repeat the step's last chunk)
  auto issue = [&](int slot, int step) {
    unsigned char* dst = &ring[slot][0];
#pragma unroll
    for (int u = 0; u < kPassStepTiles; ++u) {
      // a tile past the split's end: the split's last tile again (its keys
      // are masked; no lane reads a slot the sequence does not own)
      const int key0 = min(key_begin + (step * kPassStepTiles + u) * kTileKeys, last_key0);
      TileAddr<kUniform, false> ta;
      ta.init(a.geom, table, tlen, tc, key0);
      const int lim = last - key0;
#pragma unroll
      for (int i = 0; i < GT::kOpsPerWave; ++i) {
        const int op = wave + i * kHeads;
        const int r = op * GT::kRowsPerOp + lane / GT::kChunks;
        const int chunk = (lane % GT::kChunks) ^ GT::swz(r);
        const int64_t src = ta.at(a.geom, table, tlen, key0, min(r, lim)) + chunk * kEltPerChunk;
        lds_dma16<kCacheStream>(src_cache + src, dst + u * GT::kBytes + op * kWave * 16);
      }
    }
    if constexpr (kPass == kDecodePV) {
      const int t0 = step * kPassStepTiles;
      const int chunks = min(kPassStepTiles, ntiles - t0) * 2 * group;
      const uint16_t* src = hscores + ((int64_t)t0 * group) * kTileKeys + min(lane, chunks - 1) * kEltPerChunk;
      lds_dma16<kCacheDefault>(src, dst + kTilesBytes + wave * kWave * 16);
    }
  };

  // Per-lane LDS offsets within a tile: the K slice vectors, the V^T reads.
  uint32_t koff[F::kVec];
#pragma unroll
  for (int j = 0; j < F::kVec; ++j) koff[j] = GT::chunk_offset(row, (wave * D * Elt<T>::kBytes + 64 * j + 16 * g) >> 4);
  uint32_t vtr[D / 16];
#pragma unroll
  for (int c = 0; c < D / 16; ++c) vtr[c] = GT::vt_offset(lane, wave, c);
  // P.V pass: this lane's scores (keys 4g..4g+3 of query row `row`) of the
  // step's first and second tile in its wave's score chunk
  const uint32_t soff = kTilesBytes + wave * kWave * 16 + row * 2 * kTileKeys + 8 * g;

  constexpr int kAhead = kStages - 1;
#pragma unroll
  for (int j = 0; j < kAhead; ++j) {
    if (j < nsteps) issue(j, j);
  }

  // P.V pass: the row's (m, l) over all splits of the sequence; scores
  // pass: RoPE of q and of the new K row
  float row_m = 0.f, row_l = 1.f, row_r = 1.f;
  if constexpr (kPass == kDecodePV) {
    float m = kNegInf, l = 0.f;
    auto combine = [&](float2 v) {
      const float mn = score_max(m, v.x);
      if (mn != kNegInf) l = fmaf(l, exp_ref(m - mn), v.y * exp_ref(v.x - mn));  // one explicit fma: with two products the compiler may fuse either
      m = mn;
    };
#pragma unroll
    for (int j = 0; j < kMlBatch; ++j) combine(ml_first[j]);
    for (int64_t s0 = 4 * kMlBatch; s0 < nsplit; s0 += 4 * kMlBatch) {
      float2 v[kMlBatch];
#pragma unroll
      for (int j = 0; j < kMlBatch; ++j) {
        const int64_t sp = s0 + 4 * j + g;
        v[j] = (row_valid && sp < nsplit)
                   ? *reinterpret_cast<const float2*>(a.ws_ml + ((w.first_item + sp) * a.q_heads + qh) * 2)
                   : make_float2(kNegInf, 0.f);
      }
#pragma unroll
      for (int j = 0; j < kMlBatch; ++j) combine(v[j]);
    }
    row_m = max_over_groups(m);
    row_l = sum_over_groups(row_m == kNegInf ? 0.f : l * exp_ref(m - row_m));
    row_r = 1.f / row_l;
  } else if (rope) {
    if (row_valid) {
#pragma unroll
      for (int j = 0; j < kQHalf; ++j) {
        v4u lo = __builtin_bit_cast(v4u, qf.v[j]), hi = __builtin_bit_cast(v4u, qf.v[j + kQHalf]);
        rope_vec<T>(lo, hi, q_cos[j], q_sin[j]);
        qf.v[j] = __builtin_bit_cast(uint4, lo);
        qf.v[j + kQHalf] = __builtin_bit_cast(uint4, hi);
      }
    }
    v4u other;
#pragma unroll
    for (int k = 0; k < 4; ++k) other[k] = (uint32_t)__shfl_xor((int)new_chunk[k], kHeadChunks / 2);
    if (carrier && carries_k) {
      const bool first_half = new_c < kHeadChunks / 2;
      v4u lo = first_half ? new_chunk : other, hi = first_half ? other : new_chunk;
      rope_vec<T>(lo, hi, k_cos, k_sin);
      new_chunk = first_half ? lo : hi;
    }
  } else if (kPass == kDecodeScores && row_valid && a.rope_cos != nullptr && a.k_new != nullptr) {
    // (a split that does not end the sequence rotates q only)
#pragma unroll
    for (int j = 0; j < kQHalf; ++j) {
      v4u lo = __builtin_bit_cast(v4u, qf.v[j]), hi = __builtin_bit_cast(v4u, qf.v[j + kQHalf]);
      rope_vec<T>(lo, hi, q_cos[j], q_sin[j]);
      qf.v[j] = __builtin_bit_cast(uint4, lo);
      qf.v[j + kQHalf] = __builtin_bit_cast(uint4, hi);
    }
  }

  // scores pass: the row's running maximum and this lane's share (keys
  // 4g..4g+3 of every tile) of its sum of e^(s - m)
  float run_m = kNegInf;
  double run_l = 0.0;
  // P.V pass: O^T accumulators of the lane's row
  v4f o[D / 16];
#pragma unroll
  for (int c = 0; c < D / 16; ++c) o[c] = v4f{0.f, 0.f, 0.f, 0.f};
  bool carry = false;
  T* new_dst = nullptr;

  for (int s0 = 0; s0 < nsteps; s0 += kStages) {
#pragma unroll
    for (int j = 0; j < kStages; ++j) {
      const int st = s0 + j;
      if (st >= nsteps) break;  // uniform over the workgroup
      // this wave's ops of step st have landed once at most those of the
      // steps issued after it are outstanding; the barrier extends that to
      // every wave, and every wave has finished step st-1, whose stage the
      // next fetch reuses
      wait_dma_groups<kOwnOps, kAhead - 1>(min(kAhead - 1, nsteps - 1 - st));
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_sched_barrier(0);
      if (st + kAhead < nsteps) issue((j + kAhead) % kStages, st + kAhead);
      __builtin_amdgcn_sched_barrier(0);
      const unsigned char* stage = &ring[j][0];
      const int key0 = key_begin + st * kStepKeys;
      if constexpr (kPass == kDecodeScores) {
        if (appender && st == nsteps - 1) {
          // the new token's K row (rotated) over the stale copy the DMA
          // read from its slot, and its cache slot for both K and V
          const int pos = seq_len - 1;
          int lb, off;
          if (a.geom.bs_shift >= 0) {
            lb = pos >> a.geom.bs_shift;
            off = pos & (a.geom.block_size - 1);
          } else {
            lb = (int)((uint32_t)pos / (uint32_t)a.geom.block_size);
            off = pos - lb * a.geom.block_size;
          }
          int phys;
          if constexpr (kUniform) {
            phys = tc.template lookup<false>(table, tlen, lb);
          } else {
            phys = table[lb];
          }
          if (carrier && lb < tlen && phys >= 0 && phys < a.geom.num_blocks) {
            T* cache = reinterpret_cast<T*>(const_cast<void*>(carries_k ? a.k_cache : a.v_cache));
            new_dst = cache + a.geom.layer_offset + ((int64_t)phys * a.geom.block_size + off) * a.geom.row_elems +
                      h * D + new_c * kEltPerChunk;
            carry = true;
            if (carries_k) {
              const int rel = pos - key0;  // in [0, 32): tile rel / 16, row rel % 16
              const uint32_t patch = lds_off(stage) + (uint32_t)((rel / kTileKeys) * GT::kBytes) +
                                     (uint32_t)GT::chunk_offset(rel % kTileKeys, wave * kHeadChunks + new_c);
              asm volatile("ds_write_b128 %0, %1" : : "v"(patch), "v"(new_chunk) : "memory");
            }
          }
          asm volatile("s_waitcnt lgkmcnt(0)" : : : "memory");
        }
        __builtin_amdgcn_sched_barrier(0);
        // the step's K slices (both tiles), then S^T = K . Q^T per tile
        const uint32_t base = lds_off(stage);
        v4u kr[kPassStepTiles][F::kVec];
#pragma unroll
        for (int u = 0; u < kPassStepTiles; ++u) {
#pragma unroll
          for (int jj = 0; jj < F::kVec; ++jj) {
            asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(kr[u][jj]) : "v"(base + koff[jj]), "i"(u * GT::kBytes));
          }
        }
#pragma unroll
        for (int u = 0; u < kPassStepTiles; ++u) {
          static_assert(F::kVec == 2 || F::kVec == 4, "head_dim 64 or 128");
          if constexpr (F::kVec == 2) {
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(kr[u][0]), "+v"(kr[u][1]));
          } else {
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(kr[u][0]), "+v"(kr[u][1]), "+v"(kr[u][2]), "+v"(kr[u][3]));
          }
        }
        v4f sc[kPassStepTiles];
#pragma unroll
        for (int u = 0; u < kPassStepTiles; ++u) {
          v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int jj = 0; jj < F::kVec; ++jj) {
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kr[u][jj]),
                                                          __builtin_bit_cast(bf16x8_t, qf.v[jj]), acc, 0, 0, 0);
          }
          sc[u] = acc;
        }
        float tmax = kNegInf;
#pragma unroll
        for (int u = 0; u < kPassStepTiles; ++u) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = key0 + u * kTileKeys + 4 * g + i;
            sc[u][i] = key <= last ? scaled_score<T>(sc[u][i], a.scale) : kNegInf;
            tmax = score_max(tmax, sc[u][i]);
          }
          const int t = st * kPassStepTiles + u;
          if (ws_ok && row_valid && t < ntiles) {
            *reinterpret_cast<uint2*>(hscores + ((int64_t)t * group + row) * kTileKeys + 4 * g) =
                uint2{pack_bf16x2(sc[u][0], sc[u][1]), pack_bf16x2(sc[u][2], sc[u][3])};
          }
        }
        const float m_new = score_max(run_m, max_over_groups(tmax));
        if (m_new != kNegInf) {
          // the step's eight exponentials (v_exp_f32) summed in fp32,
          // pairwise, the steps in fp64, rescaled when the maximum moves
          if (run_m != m_new) run_l *= (double)fast_exp2((run_m - m_new) * kLog2e);
          const float nref = -m_new * kLog2e;
          float e[kPassStepTiles];
#pragma unroll
          for (int u = 0; u < kPassStepTiles; ++u) {
            float q4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) q4[i] = fast_exp2(fmaf(sc[u][i], kLog2e, nref));
            e[u] = (q4[0] + q4[1]) + (q4[2] + q4[3]);
          }
          run_l += (double)(e[0] + e[1]);
        }
        run_m = m_new;
      } else {
        // P = bf16(e^(s - m) / l) for the step's keys of the lane's row
        // (rows >= group and keys past the split's end: 0), then
        // O^T += V^T . P^T over both tiles in one 16x16x32 MFMA per 16 dims
        const uint32_t base = lds_off(stage);
        v2u sv[kPassStepTiles];
#pragma unroll
        for (int u = 0; u < kPassStepTiles; ++u) {
          // the second tile's rows follow the first tile's group rows
          asm volatile("ds_read_b64 %0, %1" : "=v"(sv[u]) : "v"(base + soff + (uint32_t)(u * group * 2 * kTileKeys)));
        }
        v2u vt[kPassStepTiles][D / 16];
#pragma unroll
        for (int u = 0; u < kPassStepTiles; ++u) {
#pragma unroll
          for (int c = 0; c < D / 16; ++c) {
            asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(vt[u][c]) : "v"(base + vtr[c]), "i"(u * GT::kBytes));
          }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(sv[0]), "+v"(sv[1]));
        v4s pb[kPassStepTiles];
#pragma unroll
        for (int u = 0; u < kPassStepTiles; ++u) {
          float p[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float x = bf16_bits_to_f32((sv[u][i / 2] >> (16 * (i % 2))) & 0xffffu);
            const int key = key0 + u * kTileKeys + 4 * g + i;
            p[i] = (row_valid && key <= last) ? div_ref(exp_ref(x - row_m), row_l, row_r) : 0.f;
          }
          pb[u] = pack_bf16x4(p[0], p[1], p[2], p[3]);
        }
        const bf16x8_t pp = join_bf16x4(pb[0], pb[1]);
#pragma unroll
        for (int c = 0; c < D / 16; c += 4) {
          asm volatile("s_waitcnt lgkmcnt(0)"
                       : "+v"(vt[0][c]), "+v"(vt[0][c + 1]), "+v"(vt[0][c + 2]), "+v"(vt[0][c + 3]));
          asm volatile("s_waitcnt lgkmcnt(0)"
                       : "+v"(vt[1][c]), "+v"(vt[1][c + 1]), "+v"(vt[1][c + 2]), "+v"(vt[1][c + 3]));
        }
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
          const bf16x8_t vv = join_bf16x4(__builtin_bit_cast(v4s, vt[0][c]), __builtin_bit_cast(v4s, vt[1][c]));
          o[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vv, pp, o[c], 0, 0, 0);
        }
      }
    }
  }

  // every fetch has been waited for (the last step's wait is vmcnt(0))
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
  if constexpr (kPass == kDecodeScores) {
    if (carry) *reinterpret_cast<v4u*>(new_dst) = new_chunk;
    // the split's (max, sum of e^(s - max)) per query head; a + b == b + a,
    // so every lane of the row forms the same sum
    double tl = run_l + __shfl_xor(run_l, 16);
    tl = tl + __shfl_xor(tl, 32);
    if (ws_ok && row_valid && g == 0) {
      *reinterpret_cast<float2*>(a.ws_ml + (item * a.q_heads + qh) * 2) = make_float2(run_m, (float)tl);
    }
  } else {
    if (!row_valid) return;
    if (nsplit == 1) {
      T* dst = reinterpret_cast<T*>(a.out) + b * a.o_sb + qh * a.o_sh + 4 * g;
#pragma unroll
      for (int c = 0; c < D / 16; ++c) store4<T>(dst + 16 * c, o[c][0], o[c][1], o[c][2], o[c][3]);
      return;
    }
    float* dst = a.ws_o + (item * a.q_heads + qh) * D + 4 * g;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      *reinterpret_cast<float4*>(dst + 16 * c) = make_float4(o[c][0], o[c][1], o[c][2], o[c][3]);
    }
  }
}

// ---------------------------------------------------------------------------
// One-launch decode with the reference's rounding point, for bf16, head_dim
// 64, block sizes that keep a 16-key tile inside one block and GQA groups of
// at most four query heads.  decode_pass_kernel's two launches hand the
// scores over through HBM; here every wave keeps its own scores on chip and
// only the splits' (max, sum) pairs and output shares cross workgroups:
//   - a wave owns one KV head of one work item and loads that head's K and V
//     rows straight into VGPRs (load_slice's operand layout) by buffer
//     loads, kFusedDepth two-tile steps ahead;
//   - the K phase forms the scores and the split's (max, sum) exactly as the
//     scores pass does, keeping the scores in the wave's LDS region (at most
//     kDecodeMaxTilesPerSplit tiles x 4 query rows x 16 keys, bf16);
//   - the wave publishes its pairs with agent-scope stores, which write
//     through to memory, waits for them, and counts itself in the (sequence,
//     KV head) counter of the workspace's control region; then it issues its
//     first V loads and waits (one lane polling) until every split of its
//     head has counted itself, reads their pairs with agent-scope loads and
//     combines them as the P.V pass does;
//   - the V phase stages each step's V rows in a 4 KiB LDS region of the
//     wave, from which the transposing reads form the V^T operands, and
//     accumulates bf16(e^(s - m) / l) . V as the P.V pass does;
//   - each split stores its share of the output rows (agent scope) and
//     counts it; the wave that counts the last share sums the shares in
//     decode_merge_kernel<kSum>'s order and clears the pair's counters.
// The waves of a workgroup meet once per kFusedDepth steps of each phase and
// otherwise run apart.  Only agent-scope atomic accesses carry data between
// workgroups, so no L2 writeback or invalidate is needed.  The waits rely on
// every workgroup of the call being resident at once (the launcher takes
// this path only when the grid fits the CUs' room for the kernel) for speed,
// not for correctness: a wait that gives up after spin_limit polls forms
// every split's (max, sum) itself from K, with the same steps and arithmetic
// as the splits, so it combines the same numbers.  Outputs and cache writes
// are bit-identical to the two launches' and the sum's.
// ---------------------------------------------------------------------------
constexpr int kFusedDim = 64;
constexpr int kFusedMaxGroup = 4;
// Two-tile steps of K (or V) loads in flight per wave: 16 KiB per wave,
// 128 KiB per CU.  Six steps measured slower (16 x 29600 tokens: 176-181 us
// against 172-176 us a call).
constexpr int kFusedDepth = 4;
constexpr int kFusedScoreBytes = (int)kDecodeMaxTilesPerSplit * kFusedMaxGroup * kTileKeys * 2;  // 16 KiB
constexpr int kFusedStageBytes = kPassStepTiles * kTileKeys * kFusedDim * 2;                       // 4 KiB
constexpr int kFusedWaveLds = kFusedScoreBytes + kFusedStageBytes;
constexpr int kFusedSpinLimit = 1 << 15;
// Cache policy of the K/V loads.  Each load instruction reads 64 of a row's
// 128 bytes (the next reads the rest), so the lines are worth keeping
// between the two: the streaming (nt) policy measured 3-8% slower.
constexpr int kFusedCachePolicy = kCacheDefault;
// The fourth word of a raw buffer resource on gfx9 (32-bit data format).
constexpr int kBufferRsrcWord3 = 0x00020000;

// This lane's two 16-byte vectors of one 16-key tile of a head (vector j =
// bytes [64j + 16 * (lane / 16), +16) of row lane % 16, at lane_off within
// the tile), by buffer loads whose range ends after the tile's `rows`
// valid keys: rows past them read as zero without a memory access, and a
// tile with no valid key reads nothing.  The loads are the compiler's (it
// counts them), so a loop can keep several tiles in flight.
__device__ __forceinline__ void load_tile_slice(v4u (&v)[2], const unsigned char* tile, int rows, int row_bytes,
                                                int lane_off) {
  const __amdgpu_buffer_rsrc_t r =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<unsigned char*>(tile), (short)0, rows * row_bytes, kBufferRsrcWord3);
  v[0] = __builtin_amdgcn_raw_buffer_load_b128(r, lane_off, 0, kFusedCachePolicy);
  v[1] = __builtin_amdgcn_raw_buffer_load_b128(r, lane_off + 64, 0, kFusedCachePolicy);
}

// Polls (one lane) until *word reaches `target`; false after `limit` polls.
// The sleep between polls (about 500 clocks) keeps thousands of waiting
// waves from crowding the lines they poll.
__device__ __forceinline__ bool wait_count(uint32_t* word, uint32_t target, int limit) {
  for (int n = 0; n < limit; ++n) {
    if (__hip_atomic_load(word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= target) return true;
    __builtin_amdgcn_s_sleep(8);
  }
  return false;
}

template <int kHeads>
__global__ __launch_bounds__(kHeads* kWave) void decode_fused_kernel(DecodeArgs a, DecodeItems items) {
  using T = bf16_t;
  constexpr int D = kFusedDim;
  using F = Frag<T, D>;
  using VT = GroupTile<T, D, 1>;  // one head's rows of a V tile
  static_assert(F::kVec == 2 && VT::kBytes * kPassStepTiles == kFusedStageBytes, "head_dim 64 layout");
  constexpr int kEltPerChunk = 16 / (int)sizeof(T);
  constexpr int kDepth = kFusedDepth;
  __shared__ __attribute__((aligned(16))) unsigned char lds[kHeads][kFusedWaveLds];

  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int g = lane >> 4;
  const int row = lane & 15;

  DecodeWork w;
  if (!decode_work(a, items, w)) return;
  // the work item in SGPRs: the loops' bounds and the buffer ranges below
  // must be known uniform, or the compiler serialises the loads over lanes
  const int64_t b = uniform64(w.b);
  const int64_t nsplit = uniform64(w.nsplit);
  const int64_t item = uniform64(w.first_item + w.split);
  w.first_item = uniform64(w.first_item);
  w.split = uniform64(w.split);
  const int seq_len = __builtin_amdgcn_readfirstlane(w.seq_len);
  const int tps = __builtin_amdgcn_readfirstlane((int)w.tps);
  const int h = (int)blockIdx.y * kHeads + wave;
  const int group = a.group;
  const int32_t* table = a.tables + b * a.table_stride;
  const int tlen = (int)a.table_stride;
  const int key_begin = (int)w.split * tps * kTileKeys;
  const int key_end = min(key_begin + tps * kTileKeys, seq_len);
  const bool row_valid = row < group;
  const int qh = h * group + row;
  const bool has_new = a.k_new != nullptr;
  const int last_key = seq_len - 1;  // the appended key, with an append
  const int row_bytes = a.geom.row_elems32 * (int)sizeof(T);
  const int lane_off = row * row_bytes + (h * D + kEltPerChunk * g) * (int)sizeof(T);
  const unsigned char* const kbytes = reinterpret_cast<const unsigned char*>(a.k_cache);
  const unsigned char* const vbytes = reinterpret_cast<const unsigned char*>(a.v_cache);
  DecodeCtl* const ctl = a.ctl;
  const int64_t pair = b * a.geom.kv_heads + h;  // (sequence, KV head)
  // the sequence's (max, sum) slots lie inside the workspace and its pair
  // has a counter (uniform); otherwise only the append is done
  const bool ws_ok = a.ws_ml != nullptr && ctl != nullptr && w.first_item + nsplit <= a.ws_items && pair < kCtlPairs;

  // q, and with an append the new K row (both rotated with RoPE) and V row
  F qf, kn, vn;
  if (row_valid) {
    load_slice<T, D>(qf, reinterpret_cast<const T*>(a.q) + b * a.q_sb + qh * a.q_sh);
  } else {
    qf.v[0] = qf.v[1] = uint4{0u, 0u, 0u, 0u};
  }
  kn.v[0] = kn.v[1] = vn.v[0] = vn.v[1] = uint4{0u, 0u, 0u, 0u};
  // append: the new rows have a slot in the pool, so they are written there
  // and their key reads them; otherwise (as kv_append skips such a slot)
  // nothing is written and the key reads what the cache holds
  bool append = false;
  if (has_new) {
    load_slice<T, D>(kn, reinterpret_cast<const T*>(a.k_new) + b * a.kn_s + h * D);
    load_slice<T, D>(vn, reinterpret_cast<const T*>(a.v_new) + b * a.vn_s + h * D);
    if (a.rope_cos != nullptr) {
      int64_t pos = last_key;
      pos = pos >= a.rope_rows ? a.rope_rows - 1 : pos;
      const int d0 = kEltPerChunk * g;  // the lane's dims 8g..8g+7 (and 32 + 8g..)
      const v4u c = *reinterpret_cast<const v4u*>(reinterpret_cast<const T*>(a.rope_cos) + pos * (D / 2) + d0);
      const v4u s = *reinterpret_cast<const v4u*>(reinterpret_cast<const T*>(a.rope_sin) + pos * (D / 2) + d0);
      v4u lo = __builtin_bit_cast(v4u, kn.v[0]), hi = __builtin_bit_cast(v4u, kn.v[1]);
      rope_vec<T>(lo, hi, c, s);
      kn.v[0] = __builtin_bit_cast(uint4, lo);
      kn.v[1] = __builtin_bit_cast(uint4, hi);
      if (row_valid) {
        lo = __builtin_bit_cast(v4u, qf.v[0]);
        hi = __builtin_bit_cast(v4u, qf.v[1]);
        rope_vec<T>(lo, hi, c, s);
        qf.v[0] = __builtin_bit_cast(uint4, lo);
        qf.v[1] = __builtin_bit_cast(uint4, hi);
      }
    }
    int lb, off;
    if (a.geom.bs_shift >= 0) {
      lb = last_key >> a.geom.bs_shift;
      off = last_key & (a.geom.block_size - 1);
    } else {
      lb = (int)((uint32_t)last_key / (uint32_t)a.geom.block_size);
      off = last_key - lb * a.geom.block_size;
    }
    const int phys = __builtin_amdgcn_readfirstlane(lb < tlen ? table[lb] : -1);
    append = phys >= 0 && phys < a.geom.num_blocks;
    // the split that ends the sequence writes the new rows to their slot
    // (row 0's lanes the K row, row 1's the V row); the loads below take
    // the new rows from registers, never from the slot
    if (append && key_end == seq_len && row < 2) {
      {
        T* cache = reinterpret_cast<T*>(const_cast<void*>(row == 0 ? a.k_cache : a.v_cache));
        uint4* dst = reinterpret_cast<uint4*>(cache + a.geom.layer_offset +
                                              ((int64_t)phys * a.geom.block_size + off) * a.geom.row_elems + h * D +
                                              kEltPerChunk * g);
        uint4 lo, hi;  // (assigned by branches: a conditional over the two rows would select their addresses)
        if (row == 0) {
          lo = kn.v[0];
          hi = kn.v[1];
        } else {
          lo = vn.v[0];
          hi = vn.v[1];
        }
        dst[0] = lo;
        dst[4] = hi;  // 64 bytes further: dims 32 + 8g..
      }
    }
  }
  if (!ws_ok) return;
  // the loads above are issued before the K loads (the loop's waits count on it)
  __builtin_amdgcn_sched_barrier(0);

  unsigned char* const scores = &lds[wave][0];  // tile t, query row n, key k at ((t * group + n) * 16 + k) * 2
  unsigned char* const vstage = &lds[wave][kFusedScoreBytes];

  // The (max, sum of e^(s - max)) of query row `row` over the keys [kb, ke)
  // (kb a multiple of 16, at most kDecodeMaxTilesPerSplit tiles, inside the
  // window of tc), formed as the scores pass forms a split's; with kKeep the
  // scores go to the wave's LDS region.
  auto split_stats = [&](auto keep, int kb, int ke, TableCache& tc) -> float2 {
    constexpr bool kKeep = decltype(keep)::value;
    const int last = ke - 1;
    const int ntiles = (ke - kb + kTileKeys - 1) / kTileKeys;
    const int nsteps = (ntiles + kPassStepTiles - 1) / kPassStepTiles;
    auto issue = [&](v4u (&dst)[kPassStepTiles][2], int st) {
#pragma unroll
      for (int u = 0; u < kPassStepTiles; ++u) {
        const int key0 = kb + (st * kPassStepTiles + u) * kTileKeys;
        TileAddr<true, false> ta;
        ta.init(a.geom, table, tlen, tc, key0);
        const int rows = key0 <= last ? min(kTileKeys, ke - key0) : 0;
        load_tile_slice(dst[u], kbytes + ta.base * (int64_t)sizeof(T), rows, row_bytes, lane_off);
      }
    };
    v4u kq[kDepth][kPassStepTiles][2];
    // in step order (the loop's waits count on it)
    static_for<0, kDepth>([&](auto j) {
      issue(kq[j], j);
      __builtin_amdgcn_sched_barrier(0);
    });
    float run_m = kNegInf;
    double run_l = 0.0;
    // step st, whose loads are in slot j = st % kDepth
    auto step = [&](auto jc, int st) {
        constexpr int j = decltype(jc)::value;
        v4u kt[kPassStepTiles][2];
#pragma unroll
        for (int u = 0; u < kPassStepTiles; ++u) {
          kt[u][0] = kq[j][u][0];
          kt[u][1] = kq[j][u][1];
        }
        const int key0 = kb + st * kPassStepTiles * kTileKeys;
        if (append && key0 <= last_key && last_key - key0 < kPassStepTiles * kTileKeys) {
          // the appended key's row from registers (its slot may not hold it yet)
#pragma unroll
          for (int u = 0; u < kPassStepTiles; ++u) {
            if (key0 + u * kTileKeys + row == last_key) {
              kt[u][0] = __builtin_bit_cast(v4u, kn.v[0]);
              kt[u][1] = __builtin_bit_cast(v4u, kn.v[1]);
            }
          }
        }
        v4f sc[kPassStepTiles];
#pragma unroll
        for (int u = 0; u < kPassStepTiles; ++u) {
          v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int jj = 0; jj < F::kVec; ++jj) {
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kt[u][jj]),
                                                          __builtin_bit_cast(bf16x8_t, qf.v[jj]), acc, 0, 0, 0);
          }
          sc[u] = acc;
        }
        // the slot's next loads only once the MFMAs have read it, so the
        // new values can take the old ones' registers (two live copies of a
        // slot would make the compiler copy in-flight registers, and wait)
        __builtin_amdgcn_sched_barrier(0);
        issue(kq[j], st + kDepth);  // steps past the range read nothing
        __builtin_amdgcn_sched_barrier(0);
        float tmax = kNegInf;
#pragma unroll
        for (int u = 0; u < kPassStepTiles; ++u) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int key = key0 + u * kTileKeys + 4 * g + i;
            sc[u][i] = key <= last ? scaled_score<T>(sc[u][i], a.scale) : kNegInf;
            tmax = score_max(tmax, sc[u][i]);
          }
          if constexpr (kKeep) {
            const int t = st * kPassStepTiles + u;
            if (row_valid && t < ntiles) {
              *reinterpret_cast<uint2*>(scores + (((t * group + row) * kTileKeys + 4 * g) << 1)) =
                  uint2{pack_bf16x2(sc[u][0], sc[u][1]), pack_bf16x2(sc[u][2], sc[u][3])};
            }
          }
        }
        const float m_new = score_max(run_m, max_over_groups(tmax));
        if (m_new != kNegInf) {
          if (run_m != m_new) run_l *= (double)fast_exp2((run_m - m_new) * kLog2e);
          const float nref = -m_new * kLog2e;
          float e[kPassStepTiles];
#pragma unroll
          for (int u = 0; u < kPassStepTiles; ++u) {
            float q4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) q4[i] = fast_exp2(fmaf(sc[u][i], kLog2e, nref));
            e[u] = (q4[0] + q4[1]) + (q4[2] + q4[3]);
          }
          run_l += (double)(e[0] + e[1]);
        }
        run_m = m_new;
    };
    // whole rounds of kDepth steps (the loop's only exit is its condition,
    // so the compiler counts the loads in flight across its back edge
    // exactly), then the rest.  In the split's own pass the waves of the
    // workgroup meet after every round: left alone, the oldest waves take
    // most of the CU's memory issue and the youngest finish far behind,
    // with the CU half idle meanwhile (all of them run the same rounds; the
    // statistics of other splits, which only some waves may form, do not
    // meet)
    int s0 = 0;
    for (; s0 + kDepth <= nsteps; s0 += kDepth) {
      static_for<0, kDepth>([&](auto j) { step(j, s0 + j); });
      if constexpr (kKeep) __builtin_amdgcn_s_barrier();
    }
    static_for<0, kDepth - 1>([&](auto j) {
      if (s0 + j < nsteps) step(j, s0 + j);
    });
    double tl = run_l + __shfl_xor(run_l, 16);
    tl = tl + __shfl_xor(tl, 32);
    return make_float2(run_m, (float)tl);
  };

  // ---- K phase: this split's scores (kept) and (max, sum) ----
  TableCache tc;
  tc.load(table, tlen, key_begin >> a.geom.bs_shift);
  const float2 own = split_stats(std::true_type{}, key_begin, key_end, tc);

  // publish: the pairs are stored through to memory before the count moves
  float* const ml = a.ws_ml + (w.first_item * a.q_heads + qh) * 2;  // this row's pair of the sequence's split 0
  if (nsplit > 1) {
    if (row_valid && g == 0) {
      __hip_atomic_store(reinterpret_cast<uint64_t*>(ml + w.split * a.q_heads * 2),
                         (uint64_t)__float_as_uint(own.x) | ((uint64_t)__float_as_uint(own.y) << 32),
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
    if (lane == 0) __hip_atomic_fetch_add(&ctl->pair[pair].count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // ---- V phase ----
  const int ntiles = (key_end - key_begin + kTileKeys - 1) / kTileKeys;
  const int nsteps = (ntiles + kPassStepTiles - 1) / kPassStepTiles;
  const int last = key_end - 1;
  auto issue_v = [&](v4u (&dst)[kPassStepTiles][2], int st) {
#pragma unroll
    for (int u = 0; u < kPassStepTiles; ++u) {
      const int key0 = key_begin + (st * kPassStepTiles + u) * kTileKeys;
      TileAddr<true, false> ta;
      ta.init(a.geom, table, tlen, tc, key0);
      const int rows = key0 <= last ? min(kTileKeys, key_end - key0) : 0;
      load_tile_slice(dst[u], vbytes + ta.base * (int64_t)sizeof(T), rows, row_bytes, lane_off);
    }
  };
  v4u vq[kDepth][kPassStepTiles][2];
  static_for<0, kDepth>([&](auto j) {
    issue_v(vq[j], j);
    __builtin_amdgcn_sched_barrier(0);
  });

  // the row's (m, l) over every split of the sequence: lane group g takes
  // splits g, g + 4, ... in order, then the groups combine (as in the P.V
  // pass)
  float m = kNegInf, l = 0.f;
  auto combine = [&](float2 v) {
    const float mn = score_max(m, v.x);
    if (mn != kNegInf) l = fmaf(l, exp_ref(m - mn), v.y * exp_ref(v.x - mn));
    m = mn;
  };
  if (nsplit == 1) {
    if (g == 0) combine(row_valid ? own : make_float2(kNegInf, 0.f));
  } else {
    // the wave waits only for its own head's splits (a wave of the
    // workgroup that is behind holds no other wave back)
    int ready = 1;
    if (lane == 0) ready = wait_count(&ctl->pair[pair].count, (uint32_t)nsplit, a.spin_limit) ? 1 : 0;
    ready = __builtin_amdgcn_readfirstlane(ready);
    if (ready) {
      constexpr int kMlBatch = 8;
      for (int64_t s0 = 0; s0 < nsplit; s0 += 4 * kMlBatch) {
        float2 v[kMlBatch];
#pragma unroll
        for (int j = 0; j < kMlBatch; ++j) {
          const int64_t sp = s0 + 4 * j + g;
          if (row_valid && sp < nsplit) {
            const uint64_t bits = __hip_atomic_load(reinterpret_cast<uint64_t*>(ml + sp * a.q_heads * 2),
                                                    __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            v[j] = make_float2(__uint_as_float((uint32_t)bits), __uint_as_float((uint32_t)(bits >> 32)));
          } else {
            v[j] = make_float2(kNegInf, 0.f);
          }
        }
#pragma unroll
        for (int j = 0; j < kMlBatch; ++j) combine(v[j]);
      }
    } else {
      // the other splits did not all arrive within the poll limit: form
      // every split's pair from K here, combining them in the same order
      if (lane == 0) __hip_atomic_fetch_add(&ctl->gave_up.count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      TableCache tcs;
      for (int64_t sp = 0; sp < nsplit; ++sp) {
        const int kb = (int)sp * tps * kTileKeys;
        const int ke = min(kb + tps * kTileKeys, seq_len);
        tcs.load(table, tlen, kb >> a.geom.bs_shift);
        const float2 v = split_stats(std::false_type{}, kb, ke, tcs);
        if ((int)(sp & 3) == g) combine(row_valid ? v : make_float2(kNegInf, 0.f));
      }
      // nothing of the K loads in flight past here (their registers are
      // free for the V phase without a wait per step)
      __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    }
  }
  const float row_m = max_over_groups(m);
  const float row_l = sum_over_groups(row_m == kNegInf ? 0.f : l * exp_ref(m - row_m));
  const float row_r = 1.f / row_l;

  v4f o[D / 16];
#pragma unroll
  for (int c = 0; c < D / 16; ++c) o[c] = v4f{0.f, 0.f, 0.f, 0.f};
  typedef __attribute__((address_space(3))) v4s lds_v4s;
  typedef __attribute__((address_space(3))) unsigned char lds_u8;
  lds_u8* const vstage_lds = (lds_u8*)vstage;
  auto vstep = [&](auto jc, int st) {
      constexpr int j = decltype(jc)::value;
      v4u vt[kPassStepTiles][2];
#pragma unroll
      for (int u = 0; u < kPassStepTiles; ++u) {
        vt[u][0] = vq[j][u][0];
        vt[u][1] = vq[j][u][1];
      }
      const int key0 = key_begin + st * kPassStepTiles * kTileKeys;
      if (append && key0 <= last_key && last_key - key0 < kPassStepTiles * kTileKeys) {
#pragma unroll
        for (int u = 0; u < kPassStepTiles; ++u) {
          if (key0 + u * kTileKeys + row == last_key) {
            vt[u][0] = __builtin_bit_cast(v4u, vn.v[0]);
            vt[u][1] = __builtin_bit_cast(v4u, vn.v[1]);
          }
        }
      }
      // the step's V rows into the wave's stage (chunk 4jj + g of row `row`)
#pragma unroll
      for (int u = 0; u < kPassStepTiles; ++u) {
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
          *reinterpret_cast<v4u*>(vstage + u * VT::kBytes + VT::chunk_offset(row, 4 * jj + g)) = vt[u][jj];
        }
      }
      // the slot's next loads once its values are staged (as in the K phase)
      __builtin_amdgcn_sched_barrier(0);
      issue_v(vq[j], st + kDepth);
      __builtin_amdgcn_sched_barrier(0);
      // the lane's scores (keys 4g..4g+3 of both tiles) and the V^T operands
      uint2 sv[kPassStepTiles];
#pragma unroll
      for (int u = 0; u < kPassStepTiles; ++u) {
        const int t = min(st * kPassStepTiles + u, ntiles - 1);
        sv[u] = *reinterpret_cast<const uint2*>(scores + (((t * group + row) * kTileKeys + 4 * g) << 1));
      }
      v4s vtr[kPassStepTiles][D / 16];
#pragma unroll
      for (int u = 0; u < kPassStepTiles; ++u) {
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
          vtr[u][c] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
              (lds_v4s*)(vstage_lds + u * VT::kBytes + VT::vt_offset(lane, 0, c)));
        }
      }
      v4s pb[kPassStepTiles];
#pragma unroll
      for (int u = 0; u < kPassStepTiles; ++u) {
        const uint32_t sw[2] = {sv[u].x, sv[u].y};
        float p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float x = bf16_bits_to_f32((sw[i / 2] >> (16 * (i % 2))) & 0xffffu);
          const int key = key0 + u * kTileKeys + 4 * g + i;
          p[i] = (row_valid && key <= last) ? div_ref(exp_ref(x - row_m), row_l, row_r) : 0.f;
        }
        pb[u] = pack_bf16x4(p[0], p[1], p[2], p[3]);
      }
      const bf16x8_t pp = join_bf16x4(pb[0], pb[1]);
#pragma unroll
      for (int c = 0; c < D / 16; ++c) {
        o[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(join_bf16x4(vtr[0][c], vtr[1][c]), pp, o[c], 0, 0, 0);
      }
  };
  // whole rounds of kDepth steps, then the rest (as in the K phase, the
  // waves meet after every round)
  int s0 = 0;
  for (; s0 + kDepth <= nsteps; s0 += kDepth) {
    static_for<0, kDepth>([&](auto j) { vstep(j, s0 + j); });
    __builtin_amdgcn_s_barrier();
  }
  static_for<0, kDepth - 1>([&](auto j) {
    if (s0 + j < nsteps) vstep(j, s0 + j);
  });

  if (nsplit == 1) {
    if (!row_valid) return;
    T* dst = reinterpret_cast<T*>(a.out) + b * a.o_sb + qh * a.o_sh + 4 * g;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) store4<T>(dst + 16 * c, o[c][0], o[c][1], o[c][2], o[c][3]);
    return;
  }
  // the split's share of each row, through to memory; the wave that counts
  // the pair's last share sums them (in decode_merge_kernel<kSum>'s order)
  // and starts the pair's counters over: every split of the pair has passed
  // its wait by then (each counts its share after its wait)
  if (row_valid) {
    float* dst = a.ws_o + (item * a.q_heads + qh) * D + 4 * g;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) store_agent4(dst + 16 * c, o[c][0], o[c][1], o[c][2], o[c][3]);
  }
  asm volatile("s_waitcnt vmcnt(0)" : : : "memory");
  uint32_t before = 0;
  if (lane == 0) before = __hip_atomic_fetch_add(&ctl->pair[pair].done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  before = __builtin_amdgcn_readfirstlane(before);
  if (before != (uint32_t)nsplit - 1u) return;
  sum_rows<T, D, true, kFusedMaxGroup>(a.ws_o + (w.first_item * a.q_heads + h * group) * D, D, (int64_t)a.q_heads * D,
                                      (int)nsplit, group, reinterpret_cast<T*>(a.out) + b * a.o_sb + h * group * a.o_sh,
                                      a.o_sh);
  if (lane == 0) {
    __hip_atomic_store(&ctl->pair[pair].count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&ctl->pair[pair].done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Split merge: one wave per (sequence, query head); sequences with a single
// split were finished by the decode kernel.  The sequence's first item is
// the sum of the split counts of the sequences before it.
constexpr int kMergeWaves = 4;

// kSum: the partials of the two-pass rounding (summed, not weighted).
template <typename T, int D, bool kSum>
__global__ __launch_bounds__(kMergeWaves* kWave) void decode_merge_kernel(DecodeArgs a, DecodeItems items) {
  const int64_t b = blockIdx.x;
  const int qh = (int)blockIdx.y * kMergeWaves + (int)(threadIdx.x / kWave);
  if (qh >= a.q_heads) return;
  int64_t nsplit, first = 0;
  if (a.dev_items != nullptr && a.dev_items->count > 0) {
    const DecodeItems* __restrict__ d = a.dev_items;
    nsplit = cdiv(cdiv((int64_t)d->seq_len[b], (int64_t)kTileKeys), (int64_t)d->tps);
    first = d->seq_first[b];
  } else if (items.count > 0) {
    nsplit = cdiv(cdiv((int64_t)items.seq_len[b], (int64_t)kTileKeys), (int64_t)a.tiles_per_split);
    first = items.seq_first[b];
  } else {
    int first_len;
    const int64_t tps = decode_call_tps(a, &first_len);
    // lane b already holds the length of one of the first 64 sequences
    const int64_t len_b = b < kWave ? __shfl(first_len, (int)b) : a.seq_lens[b];
    nsplit = len_b > 0 ? cdiv(cdiv(len_b, (int64_t)kTileKeys), tps) : (int64_t)0;
    for (int64_t s = lane_id(); s < b; s += kWave) first += decode_splits_of(a, s, tps, first_len);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) first += __shfl_xor(first, off);
  }
  if (nsplit <= 1) return;
  if (first + nsplit > a.ws_items) return;
  if constexpr (kSum) {
    sum_row<T, D>(a.ws_o + (first * a.q_heads + qh) * D, (int64_t)a.q_heads * D, (int)nsplit,
                  reinterpret_cast<T*>(a.out) + b * a.o_sb + qh * a.o_sh);
    return;
  }
  merge_row<T, D>(a.ws_o + (first * a.q_heads + qh) * D, (int64_t)a.q_heads * D,
                  a.ws_ml + (first * a.q_heads + qh) * 2, (int64_t)a.q_heads * 2, (int)nsplit,
                  reinterpret_cast<T*>(a.out) + b * a.o_sb + qh * a.o_sh);
}

// Work decomposition of a decode call.  A workgroup costs about
// kDecodeFixedTiles tile-times of fixed latency (lengths -> block table ->
// first DMA, and the drain at the end) plus one tile-time per 16-key tile,
// and the workgroups of a call run in rounds of (CUs x resident workgroups
// per CU).  The planner takes the number of rounds r that minimises
// r * (kDecodeFixedTiles + tiles per split), where tiles per split is the
// smallest that fits the call into r rounds, within [4, 128] (128 = the
// per-split block-table window, two VGPRs per lane).
constexpr int64_t kDefaultCUs = 256;  // MI355X, when the device cannot be queried

// Compute units of the current device (hipDeviceAttributeMultiprocessorCount),
// queried once per device; kDefaultCUs when there is no device to ask (the
// workspace queries also run on hosts without a GPU).
int64_t device_cus() {
  constexpr int kMaxDev = 64;
  static std::atomic<int> cached[kMaxDev] = {};
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) {
    (void)hipGetLastError();
    return kDefaultCUs;
  }
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
      (void)hipGetLastError();
      n = (int)kDefaultCUs;
    }
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

static_assert(kDecodeMaxTilesPerSplit == kTableWindow, "a split's blocks fit the block-table window");
constexpr int64_t kDecodeFixedTiles = 4;
constexpr int64_t kDecodeMaxRounds = 8;

// Tuning overrides: NIE_DECODE_MAX_HEADS caps the KV heads per workgroup,
// NIE_DECODE_TILES_PER_SPLIT fixes the split length.
int env_int(const char* name) {
  const char* env = getenv(name);
  return env ? atoi(env) : 0;
}

int decode_heads_cap() {
  static const int cap = env_int("NIE_DECODE_MAX_HEADS");
  return cap > 0 ? cap : 1 << 30;
}

int64_t decode_tiles_override() {
  static const int64_t tps = env_int("NIE_DECODE_TILES_PER_SPLIT");
  return tps;
}

struct DecodePlan {
  int heads = 1;      // KV heads per workgroup (one wave each)
  int resident = 1;   // workgroups resident on one CU
  int64_t slots = 1;  // workgroups of one round: CUs x resident / head groups
  int64_t tps = 0;    // 16-key tiles per split; 0: chosen on the device (decode_device_tps)
  int64_t items = 0;  // grid.x: an upper bound on the number of work items
};

// Workspace layout of a decode call: the partial O rows (items x q_heads x
// head_dim floats), then (max, sum) pairs (items x q_heads x 2 floats).
int64_t decode_max_items(int64_t batch, int64_t total_seq_len, int64_t tps) {
  // sum_b ceil(ceil(len_b/16)/tps) <= (sum_b len_b/16 + batch)/tps + batch
  return (cdiv(total_seq_len, kTileKeys) + batch) / tps + batch + 1;
}

// Rounding point of the bf16 attention probabilities, process-wide
// (nie_set_attention_rounding): NIE_ROUND_REFERENCE, the reference's (two
// passes), or NIE_ROUND_FAST (one pass, online softmax).
std::atomic<int> g_rounding{NIE_ROUND_REFERENCE};

bool two_pass(int dtype) {
  return dtype == NIE_DTYPE_BF16 && g_rounding.load(std::memory_order_relaxed) == NIE_ROUND_REFERENCE;
}

// Key slots (16 per tile of every item) of the two-pass score buffer: items
// x tps x 16.  With the split length chosen on the device (tps 0) the items
// of a sequence cover at most its tiles + tps - 1 slots' worth of tiles, so
// items x tps <= sum of tiles + batch x (kDecodeMaxTilesPerSplit - 1).
int64_t decode_score_keys(const DecodePlan& p, int64_t batch, int64_t total_seq_len) {
  if (p.tps > 0) return p.items * p.tps * kTileKeys;
  return (cdiv(total_seq_len, kTileKeys) + batch * kDecodeMaxTilesPerSplit) * kTileKeys;
}

// Workspace of a decode call: the partial O rows (items x q_heads x head_dim
// floats), the (max, sum) pairs (items x q_heads x 2 floats), and with the
// two-pass rounding the scores (key slots x q_heads bf16), 256-byte aligned.
int64_t decode_ws_partials(const DecodePlan& p, int64_t q_heads, int64_t head_dim) {
  return (p.items * q_heads * (head_dim + 2) * (int64_t)sizeof(float) + 255) / 256 * 256;
}

int64_t decode_workspace_need(const DecodePlan& p, int64_t q_heads, int64_t head_dim, int64_t batch,
                              int64_t total_seq_len, bool two) {
  const int64_t partials = p.items * q_heads * (head_dim + 2) * (int64_t)sizeof(float);
  if (!two) return partials;
  return decode_ws_partials(p, q_heads, head_dim) + decode_score_keys(p, batch, total_seq_len) * q_heads * 2;
}

// ---------------------------------------------------------------------------
// Attention for shapes the MFMA kernels are not built for (any head_dim up to
// kGenericMaxDim, any GQA group): one wave per (query row, query head), the
// lanes over the head dims.  Two passes over the keys keep the reference's
// rounding points exactly: pass 1 forms the running maximum and the fp32
// softmax denominator of the scores (q.k rounded to the storage dtype, times
// the scale, rounded again: layers/paged_attention.py:97-98,
// layers/attention.py:400); pass 2 recomputes each score and accumulates
// round(exp(s - m) / l) * v in fp32 (the probabilities cast to the storage
// dtype before P.V, :109-114 and :410-411), rounding once at the end.  The
// work per key is a wave reduction, so these shapes run far below the tuned
// kernels' rate; they exist so that every shape the reference accepts runs.
// ---------------------------------------------------------------------------
constexpr int kGenericMaxDim = 256;
constexpr int kGenericWaves = 4;

struct GenericAttnArgs {
  const void* q;
  int64_t q_sr, q_sh;  // query row / head strides (elements)
  void* out;
  int64_t o_sr, o_sh;
  const void* k_cache;
  const void* v_cache;
  CacheGeom geom;
  int32_t head_dim;
  int32_t q_heads;
  int32_t group;
  const int32_t* tables;
  int64_t table_stride;
  float scale;
  int64_t rows;  // query rows
  // decode: row b is sequence b over its first seq_lens[b] keys
  const int32_t* seq_lens;
  // varlen (seq_lens == nullptr): row t of request r (cu_seqlens[r] <= t <
  // cu_seqlens[r + 1]) sees keys [0, context_lens[r] + t - cu_seqlens[r]]
  const int64_t* cu_seqlens;
  const int32_t* context_lens;
  int64_t num_seqs;
  // decode only: RoPE of q at position seq_len - 1 (cos / sin tables
  // (rope_rows, head_dim / 2)); nullptr: none
  const void* rope_cos;
  const void* rope_sin;
  int64_t rope_rows;
};

__device__ __forceinline__ float wave_sum_f32(float x) {
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) x += __shfl_xor(x, off);
  return x;
}

template <typename T>
__global__ __launch_bounds__(kGenericWaves* kWave) void attention_generic_kernel(GenericAttnArgs a) {
  constexpr int kPer = kGenericMaxDim / kWave;
  const int lane = lane_id();
  const int64_t w = (int64_t)blockIdx.x * kGenericWaves + threadIdx.x / kWave;
  if (w >= a.rows * a.q_heads) return;  // uniform over the wave
  const int64_t row = w / a.q_heads;
  const int h = (int)(w - row * a.q_heads);
  const int D = a.head_dim;
  int64_t seq;
  int nkeys;
  if (a.seq_lens != nullptr) {
    seq = row;
    nkeys = a.seq_lens[row];
  } else {
    int64_t lo = 0, hi = a.num_seqs - 1;  // the last request whose first row is <= row
    while (lo < hi) {
      const int64_t mid = (lo + hi + 1) / 2;
      if (a.cu_seqlens[mid] <= row) lo = mid;
      else hi = mid - 1;
    }
    seq = lo;
    nkeys = a.context_lens[lo] + (int)(row - a.cu_seqlens[lo]) + 1;
  }
  nkeys = __builtin_amdgcn_readfirstlane(nkeys);
  seq = uniform64(seq);
  T* orow = reinterpret_cast<T*>(a.out) + row * a.o_sr + (int64_t)h * a.o_sh;
  if (nkeys <= 0) {  // nothing to attend: zeros, not garbage
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      if (lane + kWave * i < D) store_elt<T>(orow + lane + kWave * i, 0.f);
    }
    return;
  }
  // this lane's dims of q (rotated first when RoPE tables are given)
  const T* qrow = reinterpret_cast<const T*>(a.q) + row * a.q_sr + (int64_t)h * a.q_sh;
  float q[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int d = lane + kWave * i;
    q[i] = d < D ? load_elt<T>(qrow, d) : 0.f;
    if (a.rope_cos != nullptr && d < D) {
      const int half = D / 2;
      int64_t pos = nkeys - 1;
      pos = pos >= a.rope_rows ? a.rope_rows - 1 : pos;
      const int j = d < half ? d : d - half;
      const float c = load_elt<T>(a.rope_cos, pos * half + j);
      const float sn = load_elt<T>(a.rope_sin, pos * half + j);
      const float other = load_elt<T>(qrow, d < half ? d + half : d - half);
      q[i] = d < half ? sub_t<T>(mul_t<T>(q[i], c), mul_t<T>(other, sn))
                      : add_t<T>(mul_t<T>(q[i], c), mul_t<T>(other, sn));
    }
  }
  const int32_t* table = a.tables + seq * a.table_stride;
  const int tlen = (int)a.table_stride;
  const int kvh = h / a.group;
  const T* kc = reinterpret_cast<const T*>(a.k_cache) + (int64_t)kvh * D;
  const T* vc = reinterpret_cast<const T*>(a.v_cache) + (int64_t)kvh * D;
  auto score = [&](int64_t off) {
    float part = 0.f;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int d = lane + kWave * i;
      if (d < D) part = fmaf(q[i], load_elt<T>(kc + off, d), part);
    }
    return scaled_score<T>(wave_sum_f32(part), a.scale);
  };
  float m = kNegInf, l = 0.f;
  for (int k = 0; k < nkeys; ++k) {
    const float sc = score(token_offset(a.geom, table, tlen, k));
    const float m_new = score_max(m, sc);
    l = (m == kNegInf ? 0.f : l * expf(m - m_new)) + expf(sc - m_new);
    m = m_new;
  }
  float o[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) o[i] = 0.f;
  const float inv_l = 1.f / l;
  for (int k = 0; k < nkeys; ++k) {
    const int64_t off = token_offset(a.geom, table, tlen, k);
    const float p = round_storage<T>(expf(score(off) - m) * inv_l);
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int d = lane + kWave * i;
      if (d < D) o[i] = fmaf(p, load_elt<T>(vc + off, d), o[i]);
    }
  }
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    if (lane + kWave * i < D) store_elt<T>(orow + lane + kWave * i, o[i]);
  }
}

// The fused decode step's cache write for the shapes above: sequence b's new
// K (rotated at position seq_lens[b] - 1 when RoPE tables are given, as
// rope_kv_append_kernel rotates it) and V rows into the slot its table gives;
// a table entry outside the pool skips the write.  One thread per
// (sequence, KV head, dim).
struct GenericAppendArgs {
  const void* k_new;
  int64_t kn_s;
  const void* v_new;
  int64_t vn_s;
  void* k_cache;
  void* v_cache;
  CacheGeom geom;
  int32_t head_dim;
  const int32_t* tables;
  int64_t table_stride;
  const int32_t* seq_lens;
  int64_t batch;
  const void* rope_cos;
  const void* rope_sin;
  int64_t rope_rows;
};

template <typename T>
__global__ __launch_bounds__(256) void decode_append_generic_kernel(GenericAppendArgs a) {
  const int D = a.head_dim;
  const int64_t per_seq = (int64_t)a.geom.kv_heads * D;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= a.batch * per_seq) return;
  const int64_t b = i / per_seq;
  const int64_t e = i - b * per_seq;  // element (kv head * D + dim) of the row
  const int d = (int)(e % D);
  const int pos = a.seq_lens[b] - 1;
  if (pos < 0) return;
  int lb, off;
  if (a.geom.bs_shift >= 0) {
    lb = pos >> a.geom.bs_shift;
    off = pos & (a.geom.block_size - 1);
  } else {
    lb = pos / a.geom.block_size;
    off = pos - lb * a.geom.block_size;
  }
  if (lb >= a.table_stride) return;
  const int phys = a.tables[b * a.table_stride + lb];
  if (phys < 0 || phys >= a.geom.num_blocks) return;
  const int64_t dst = a.geom.layer_offset + ((int64_t)phys * a.geom.block_size + off) * a.geom.row_elems + e;
  const T* krow = reinterpret_cast<const T*>(a.k_new) + b * a.kn_s;
  const T* vrow = reinterpret_cast<const T*>(a.v_new) + b * a.vn_s;
  float kv = load_elt<T>(krow, e);
  if (a.rope_cos != nullptr) {
    const int half = D / 2;
    int64_t rp = pos >= a.rope_rows ? a.rope_rows - 1 : pos;
    const int j = d < half ? d : d - half;
    const float c = load_elt<T>(a.rope_cos, rp * half + j);
    const float sn = load_elt<T>(a.rope_sin, rp * half + j);
    const float other = load_elt<T>(krow, d < half ? e + half : e - half);
    kv = d < half ? sub_t<T>(mul_t<T>(kv, c), mul_t<T>(other, sn)) : add_t<T>(mul_t<T>(kv, c), mul_t<T>(other, sn));
  }
  store_elt<T>(reinterpret_cast<T*>(a.k_cache) + dst, kv);
  reinterpret_cast<T*>(a.v_cache)[dst] = reinterpret_cast<const T*>(vrow)[e];
}

// rope_kv_append_kernel for an even head_dim the kernel is not built for:
// one thread per (token, head, pair index), the same per-op rounding.
template <typename T>
__global__ __launch_bounds__(256) void rope_kv_append_generic_kernel(RopeAppendArgs a, int head_dim) {
  const int half = head_dim / 2;
  const int heads = a.q_heads + 2 * a.kv_heads;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= a.num_tokens * heads * half) return;
  const int64_t r = idx / half;
  const int i = (int)(idx - r * half);
  const int64_t t = r / heads;
  const int j = (int)(r - t * heads);
  int64_t pos = a.positions[t];
  pos = pos < 0 ? 0 : (pos >= a.table_rows ? a.table_rows - 1 : pos);
  const float c = load_elt<T>(a.cos_table, pos * half + i);
  const float s = load_elt<T>(a.sin_table, pos * half + i);
  if (j < a.q_heads) {
    T* x = reinterpret_cast<T*>(a.q) + t * a.q_st + (int64_t)j * a.q_sh;
    const float x1 = load_elt<T>(x, i);
    const float x2 = load_elt<T>(x, i + half);
    store_elt<T>(x + i, sub_t<T>(mul_t<T>(x1, c), mul_t<T>(x2, s)));
    store_elt<T>(x + i + half, add_t<T>(mul_t<T>(x2, c), mul_t<T>(x1, s)));
    return;
  }
  const int64_t slot = a.slots[t];
  if (slot < 0 || slot >= a.pool_slots) return;
  const bool is_k = j < a.q_heads + a.kv_heads;
  const int h = is_k ? j - a.q_heads : j - a.q_heads - a.kv_heads;
  const int64_t dst_off = a.layer_offset + (slot * a.kv_heads + h) * head_dim;
  if (is_k) {
    const T* x = reinterpret_cast<const T*>(a.k) + t * a.k_st + (int64_t)h * a.k_sh;
    const float x1 = load_elt<T>(x, i);
    const float x2 = load_elt<T>(x, i + half);
    T* dst = reinterpret_cast<T*>(a.k_cache) + dst_off;
    store_elt<T>(dst + i, sub_t<T>(mul_t<T>(x1, c), mul_t<T>(x2, s)));
    store_elt<T>(dst + i + half, add_t<T>(mul_t<T>(x2, c), mul_t<T>(x1, s)));
  } else {
    const T* x = reinterpret_cast<const T*>(a.v) + t * a.v_st + (int64_t)h * a.v_sh;
    T* dst = reinterpret_cast<T*>(a.v_cache) + dst_off;
    dst[i] = x[i];
    dst[i + half] = x[i + half];
  }
}

// ---------------------------------------------------------------------------
// Varlen prefill
// ---------------------------------------------------------------------------
constexpr int kPrefillWaves = 4;
// Block-table windows (kTableWindow entries each, two VGPRs per window) a
// prefill wave holds: a piece covers up to 640 key tiles (10240 keys at
// block size 16), so a chunk on an 8192-token context is one piece.
constexpr int kPrefillTableWindows = 5;
constexpr int kPrefillLdsBudget = 128 * 1024;

// Query rows per wave: kRowBlocks MFMA row blocks of 16 rows, each block
// = 16/G consecutive tokens x the G query heads of the workgroup's KV head.
template <int kRowBlocks>
constexpr int prefill_rows_per_item() {
  return kPrefillWaves * kRowBlocks * 16;
}

struct PrefillArgs {
  const void* q;
  int64_t q_st, q_sh;
  const int64_t* cu_seqlens;
  const int32_t* context_lens;
  int64_t num_seqs;
  const void* k_cache;
  const void* v_cache;
  CacheGeom geom;
  int32_t group;
  int32_t tokens_per_tile;  // query tokens per work item
  int32_t tiles_per_split;  // 16-key tiles per work item
  const int32_t* tables;
  int64_t table_stride;
  float scale;
  void* out;
  int64_t o_st, o_sh;
  float* ws_o;       // (ws_items, kv_heads, rows_per_item, head_dim)
  float* ws_ml;      // (ws_items, kv_heads, rows_per_item, 2)
  int64_t ws_items;  // item slots in the workspace
  int32_t grid_items;   // prefill launch: items per KV head (1-D grid of grid_items * kv_heads)
  int32_t merge_tiles;  // merge launch: query tiles per KV head
  // The reference rounding's stats pass cuts each piece's keys into
  // stats_parts parts (1 or 2, workgroups of their own), each with its
  // (max, sum) slot: slot (first item of the tile + piece) * stats_parts +
  // part, of ws_ml_slots; the exact pass combines a tile's parts in order.
  int32_t stats_parts = 1;
  int64_t ws_ml_slots = 0;
};

// Key tiles visible to query tile qt of request r (its last row's position + 1).
__device__ __forceinline__ int prefill_key_tiles(int ctx, int q_len, int tpt, int qt) {
  const int t_end = min((qt + 1) * tpt, q_len);
  return (ctx + t_end + kTileKeys - 1) / kTileKeys;
}

// Work items (query tile, key split) of a request with q_len query tokens
// after ctx cached ones.
// Walks the query tiles of one request in order, keeping the piece count
// ceil(key tiles / S) of the current tile without a division per tile: the
// key tiles a tile sees grow by at most ceil(tpt / 16) + 1 from one tile to
// the next, so the count catches up by a few additions of S.  (A call too
// large for the host schedule has up to thousands of query tiles, and two
// integer divisions per tile in every workgroup's locate cost more VALU
// time than its attention steps.)
struct SplitWalk {
  int q_len, ctx, tpt, S;
  int t_end;   // query tokens up to the end of the current tile
  int nsplit;  // pieces of the current tile: ceil(key tiles / S)
  int cap;     // nsplit * S
  __host__ __device__ __forceinline__ void start(int q_len_, int ctx_, int tpt_, int S_) {
    q_len = q_len_;
    ctx = ctx_;
    tpt = tpt_;
    S = S_;
    t_end = min(tpt, q_len);
    nsplit = ((ctx + t_end + kTileKeys - 1) / kTileKeys + S - 1) / S;
    cap = nsplit * S;
  }
  __host__ __device__ __forceinline__ void next() {
    t_end = min(t_end + tpt, q_len);
    const int kt = (ctx + t_end + kTileKeys - 1) / kTileKeys;
    while (kt > cap) {
      cap += S;
      ++nsplit;
    }
  }
};

// Items of query tiles [0, count) of a request.  When the request's last
// query tile (which sees the most keys) fits one piece, every tile is one
// item and no walk is needed (a 2048-token prompt has 64 query tiles, and
// the walk over them cost each workgroup about a third of its VALU work).
__device__ __forceinline__ int prefill_items_upto(int q_len, int ctx, int tpt, int S, int count) {
  if ((ctx + q_len + kTileKeys - 1) / kTileKeys <= S) return count;
  SplitWalk w;
  w.start(q_len, ctx, tpt, S);
  int n = 0;
  for (int qt = 0; qt < count; ++qt) {
    if (qt > 0) w.next();
    n += w.nsplit;
  }
  return n;
}

__device__ __forceinline__ int prefill_items_of_len(int q_len, int ctx, int tpt, int S) {
  return prefill_items_upto(q_len, ctx, tpt, S, (q_len + tpt - 1) / tpt);
}

__device__ __forceinline__ int64_t prefill_items_of(const PrefillArgs& a, int64_t r) {
  const int q_len = (int)(a.cu_seqlens[r + 1] - a.cu_seqlens[r]);
  return prefill_items_of_len(q_len, a.context_lens[r], a.tokens_per_tile, a.tiles_per_split);
}

// The request of work item `item` (wave-uniform): like locate_item over
// prefill_items_of, but each lane keeps its request's lengths from the scan,
// so the found request's query start, length and context come out of the
// lanes instead of another round trip to memory.
struct PrefillItem {
  int64_t r;        // request, -1 past the last item
  int64_t local;    // item index within the request
  int64_t first;    // the request's first item
  int64_t q_begin;  // the request's first packed query row
  int q_len;
  int ctx;
};

__device__ __forceinline__ PrefillItem prefill_locate(const PrefillArgs& a, int64_t item) {
  const int lane = lane_id();
  PrefillItem it;
  int64_t base = 0;
  for (int64_t b0 = 0; b0 < a.num_seqs; b0 += kWave) {
    const int64_t b = b0 + lane;
    int64_t qb = 0;
    int qn = 0, cx = 0;
    int64_t n = 0;
    if (b < a.num_seqs) {
      qb = a.cu_seqlens[b];
      qn = (int)(a.cu_seqlens[b + 1] - qb);
      cx = a.context_lens[b];
      n = prefill_items_of_len(qn, cx, a.tokens_per_tile, a.tiles_per_split);
    }
    int64_t incl = n;  // inclusive prefix sum over the wave
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const int64_t up = __shfl_up(incl, off);
      if (lane >= off) incl += up;
    }
    const int64_t excl = incl - n;
    const int64_t total = __shfl(incl, kWave - 1);
    if (item < base + total) {
      const bool mine = (b < a.num_seqs) && (item >= base + excl) && (item < base + incl);
      const int src = __builtin_ctzll(__ballot(mine));
      it.r = (int64_t)__builtin_amdgcn_readfirstlane((int)(b0 + src));
      it.first = uniform64(base + __shfl(excl, src));
      it.local = uniform64(item) - it.first;
      it.q_begin = uniform64(__shfl(qb, src));
      it.q_len = __builtin_amdgcn_readfirstlane(__shfl(qn, src));
      it.ctx = __builtin_amdgcn_readfirstlane(__shfl(cx, src));
      return it;
    }
    base += total;
  }
  it.r = -1;
  it.local = it.first = it.q_begin = 0;
  it.q_len = it.ctx = 0;
  return it;
}

// Work items of a prefill call planned from host metadata, passed by value
// as a kernel argument: item i (one workgroup per KV head) is piece p of
// query tile k, key tiles [item_begin[i], item_begin[i] + len), with
// item[i] = k | p << 8 | len << 16; the tile's request, rows and context are
// listed per tile.  Every field is a 32-bit word, so a workgroup reads its
// item and then its tile with scalar loads.  Without the table each workgroup locates its item from the
// device copies of cu_seqlens / context_lens, with pieces of tiles_per_split
// tiles.
constexpr int kMaxSchedTiles = 64;
constexpr int kMaxSchedItems = 320;

struct PrefillSchedule {
  int32_t count = 0;  // items; 0: located on the device
  uint32_t item[kMaxSchedItems];        // tile | piece << 8 | len << 16
  uint32_t item_begin[kMaxSchedItems];  // first key tile of the piece
  uint32_t tile[kMaxSchedTiles];        // request | pieces << 8 | first item << 16 (pieces 1: rows written out)
  int32_t q_begin[kMaxSchedTiles];      // the request's first packed query row
  int32_t q_len[kMaxSchedTiles];        // the request's query tokens
  int32_t ctx[kMaxSchedTiles];          // the request's cached tokens
  int32_t t0[kMaxSchedTiles];           // the tile's first query token within the request
};

static_assert(sizeof(PrefillArgs) + sizeof(PrefillSchedule) <= 4096, "prefill kernel arguments fit 4 KiB");

// Wave priority (s_setprio takes an immediate; p is wave-uniform, clamped to
// 0..3).  Two prefill workgroups resident on one CU do not progress alike at
// equal priority: the one dispatched first keeps issue priority (oldest waves
// first), and on the mixed chunked-prefill step its 6-step piece loops in
// 6.24 us while the other's takes 8.84 us.  With the priority set from the
// steps a workgroup has left, the one behind catches up (7.88 and 8.28 us,
// kernel 13.6 -> 13.1 us).
__device__ __forceinline__ void set_wave_priority(int p) {
  if (p >= 3) {
    __builtin_amdgcn_s_setprio(3);
  } else if (p == 2) {
    __builtin_amdgcn_s_setprio(2);
  } else if (p == 1) {
    __builtin_amdgcn_s_setprio(1);
  } else {
    __builtin_amdgcn_s_setprio(0);
  }
}

// Key steps of kPrefillStepTiles 16-key tiles (64 keys) stream through an LDS
// ring of prefill_stages() steps.
constexpr int kPrefillStepTiles = 4;

template <typename T, int D>
constexpr int prefill_stage_bytes() {
  return kPrefillStepTiles * 2 * GroupTile<T, D, 1>::kBytes;
}

// bf16 keeps a step's V in the ring one iteration longer than it fetches
// ahead (the step's P.V runs in the next iteration), so it takes one stage
// more: five at head_dim 64 (80 KiB, two workgroups per CU), four at 128.
template <typename T, int D>
constexpr int prefill_stages() {
  constexpr int fit = kPrefillLdsBudget / prefill_stage_bytes<T, D>();
  constexpr int want = Elt<T>::kIsBf16 ? 5 : 4;
  return fit >= want ? want : (fit >= 2 ? fit : 2);
}


// Online softmax over one key step: s[nb][t] holds the scores of sub-tile t
// for row block nb (-inf where masked); they are overwritten with the
// unnormalised probabilities exp2((s - m) * c), where c = log2(e) times the
// factor still to be applied to s (1, or the power-of-two softmax scale when
// it has been kept out of s), and m is the row's reference maximum.  The
// reference maximum is raised (rescaling O and the denominator) only when
// some row of the wave has a score more than kRescaleLog2 above it (in
// log2 units) or had no reference yet; otherwise the probabilities of the
// step are at most 2^kRescaleLog2, which fp32 sums and bf16 operands hold
// exactly as well as values below 1.  O / denominator is the same either way.
constexpr float kRescaleLog2 = 8.f;

template <int D, int kBlocks, int kSub>
__device__ __forceinline__ void softmax_step(SoftmaxState<D> (&st)[kBlocks], v4f (&s)[kBlocks][kSub], float c) {
  float m_new[kBlocks];
  bool grow = false;
#pragma unroll
  for (int nb = 0; nb < kBlocks; ++nb) {
    float tm[kSub];
#pragma unroll
    for (int t = 0; t < kSub; ++t) {
      tm[t] = score_max(score_max(s[nb][t][0], s[nb][t][1]), score_max(s[nb][t][2], s[nb][t][3]));
    }
#pragma unroll
    for (int w = 1; w < kSub; w <<= 1) {
#pragma unroll
      for (int t = 0; t + w < kSub; t += 2 * w) tm[t] = score_max(tm[t], tm[t + w]);
    }
    m_new[nb] = score_max(st[nb].m, max_over_groups(tm[0]));
    grow |= m_new[nb] != kNegInf && (st[nb].m == kNegInf || (m_new[nb] - st[nb].m) * c > kRescaleLog2);
  }
  if (__ballot(grow)) {
#pragma unroll
    for (int nb = 0; nb < kBlocks; ++nb) {
      // alpha = 0 for a row without a reference yet (its O and sum are 0)
      const float alpha = st[nb].m == kNegInf ? 0.f : fast_exp2((st[nb].m - m_new[nb]) * c);
      st[nb].lsum *= alpha;
#pragma unroll
      for (int d = 0; d < D / 16; ++d) st[nb].o[d] *= alpha;
      st[nb].m = m_new[nb];
    }
  }
#pragma unroll
  for (int nb = 0; nb < kBlocks; ++nb) {
    // A row with nothing unmasked so far keeps m = -inf; 0 as the reference
    // point makes its exponentials exact zeros, not NaN.
    const float nref = (st[nb].m == kNegInf) ? 0.f : -st[nb].m * c;
    float ps[kSub];
#pragma unroll
    for (int t = 0; t < kSub; ++t) {
#pragma unroll
      for (int i = 0; i < 4; ++i) s[nb][t][i] = fast_exp2(fmaf(s[nb][t][i], c, nref));
      ps[t] = (s[nb][t][0] + s[nb][t][1]) + (s[nb][t][2] + s[nb][t][3]);
    }
#pragma unroll
    for (int w = 1; w < kSub; w <<= 1) {
#pragma unroll
      for (int t = 0; t + w < kSub; t += 2 * w) ps[t] += ps[t + w];
    }
    st[nb].lsum += ps[0];
  }
}

// LDS reads of the ring whose results are waited for together (see
// ring_read_k): issue, then one lgkmcnt(0) wait that all results pass
// through.
template <int N>
__device__ __forceinline__ void ring_read_b128_n(v4u (&r)[N], const uint32_t (&addr)[N]) {
  static_assert(N % 4 == 0, "groups of four");
#pragma unroll
  for (int j = 0; j < N; ++j) asm volatile("ds_read_b128 %0, %1" : "=v"(r[j]) : "v"(addr[j]));
#pragma unroll
  for (int j = 0; j < N; j += 4) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(r[j]), "+v"(r[j + 1]), "+v"(r[j + 2]), "+v"(r[j + 3]));
  }
}

template <int N>
__device__ __forceinline__ void ring_read_tr_n(v2u (&r)[N], const uint32_t (&addr)[N]) {
  static_assert(N % 4 == 0, "groups of four");
#pragma unroll
  for (int j = 0; j < N; ++j) asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(r[j]) : "v"(addr[j]));
#pragma unroll
  for (int j = 0; j < N; j += 4) {
    asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(r[j]), "+v"(r[j + 1]), "+v"(r[j + 2]), "+v"(r[j + 3]));
  }
}

// LDS reads of the ring at immediate offsets: read i (of N) is at
// base[i % kBases] + (i / kBases) * kStride, so a step's reads need kBases
// address registers.  Waited for by the caller (lgkmcnt), like ring_read_b128_n.
template <int N, int kBases, int kStride, int I = 0>
__device__ __forceinline__ void ring_read_at(v4u* r, const uint32_t* base) {
  if constexpr (I < N) {
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r[I]) : "v"(base[I % kBases]), "i"((I / kBases) * kStride));
    ring_read_at<N, kBases, kStride, I + 1>(r, base);
  }
}

template <int N, int kBases, int kStride, int I = 0>
__device__ __forceinline__ void ring_read_tr_at(v2u* r, const uint32_t* base) {
  if constexpr (I < N) {
    asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2"
                 : "=v"(r[I])
                 : "v"(base[I % kBases]), "i"((I / kBases) * kStride));
    ring_read_tr_at<N, kBases, kStride, I + 1>(r, base);
  }
}

// One workgroup = one (request, query tile, key split) for one KV head.
// Wave w owns kRowBlocks MFMA row blocks of 16 query rows (16/G consecutive
// tokens x the G query heads of the KV head each).  The head's K and V rows
// stream through an LDS ring in steps of 64 keys (four 16-key tiles), fetched
// by LDS DMA (as in decode) with the step's DMA ops spread evenly over the
// waves; every wave applies each step to all of its row blocks: four QK tiles
// per row block, one softmax over the step, and P.V in 16x16x32 MFMAs that
// each cover two 16-key tiles (bf16).  Row blocks whose tokens all precede
// the step skip it (causal mask).  With one split the rows are written out;
// with several, the split's unnormalised partial goes to the workspace for
// prefill_merge_kernel.
// kPow2Scale: the softmax scale is a power of two, so rounding the scaled
// score to bf16 is exact and the scale can be kept out of the scores and
// applied inside the exponential (bf16 only).
// kMode: kPrefillOnline, the one-pass online softmax (bf16 P =
// exp(s - running max), O / l at the end); or, with the reference's
// rounding point (normalised probabilities rounded to bf16 before P.V,
// layers/attention.py:410-411), kPrefillStats then kPrefillExact over the
// same work items.  kPrefillStats reads K only and writes, per piece and
// query row, the maximum of its scores and the sum of e^(s - max) (each
// step's exponentials summed in fp32, the steps in fp64) into the (max,
// sum) slots of the workspace; kPrefillExact combines the pieces of its
// query tile into the row's (m, l), and accumulates P = bf16(e^(s - m) / l)
// . V: with one piece the rows are written out, with several each piece's
// share of the normalised output goes to the workspace, which
// prefill_merge_kernel<kSum> adds up.
constexpr int kPrefillOnline = 0;
constexpr int kPrefillStats = 1;
constexpr int kPrefillExact = 2;

// kWindows: block-table windows a wave holds (see TableWindows): 1, or
// kPrefillTableWindows for plans with pieces longer than one window.
template <typename T, int D, bool kUniform, int kRowBlocks, bool kPow2Scale, int kMode, int kWindows>
__global__ __launch_bounds__(kPrefillWaves* kWave) __attribute__((amdgpu_waves_per_eu(2)))
void varlen_prefill_kernel(PrefillArgs a, PrefillSchedule sc) {
  using F = Frag<T, D>;
  using GT = GroupTile<T, D, 1>;
  static_assert(kMode == kPrefillOnline || Elt<T>::kIsBf16, "the reference rounding point matters for bf16");
  constexpr bool kFetchV = kMode != kPrefillStats;
  constexpr int kSub = kPrefillStepTiles;
  constexpr int kStages = prefill_stages<T, D>();
  // the stats pass stages K only: half the LDS, so more of its workgroups
  // fit a CU
  constexpr int kStageBytes = kFetchV ? prefill_stage_bytes<T, D>() : prefill_stage_bytes<T, D>() / 2;
  // DMA ops of one step: per tile, K ops then V ops (the stats pass: K only)
  constexpr int kStepOps = kSub * (kFetchV ? 2 : 1) * GT::kOps;
  static_assert(kStepOps % kPrefillWaves == 0, "step DMA ops must spread evenly over the waves");
  constexpr int kOwnOps = kStepOps / kPrefillWaves;
  constexpr int kEltPerChunk = 16 / Elt<T>::kBytes;
  constexpr int kRows = prefill_rows_per_item<kRowBlocks>();
  __shared__ __attribute__((aligned(16))) unsigned char ring[kStages][kStageBytes];

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int g = lane >> 4;
  const int row = lane & 15;
  const int tpt = a.tokens_per_tile;
  const int S = a.tiles_per_split;
  // (item, KV head) of this workgroup, head-major over the XCDs; 32-bit
  // and scalar, so the schedule below is read with scalar loads
  // (the stats pass: parts of items, consecutive)
  const int parts = kMode == kPrefillStats ? __builtin_amdgcn_readfirstlane(a.stats_parts) : 1;
  const uint32_t grid_parts = (uint32_t)a.grid_items * (uint32_t)parts;
  const uint32_t logical = xcd_logical32(blockIdx.x, grid_parts * (uint32_t)a.geom.kv_heads);
  const int h = __builtin_amdgcn_readfirstlane((int)(logical / grid_parts));
  const int wg_part = __builtin_amdgcn_readfirstlane((int)(logical - (uint32_t)h * grid_parts));
  const int wg_item = parts == 1 ? wg_part : wg_part >> 1;
  const int part = wg_part - wg_item * parts;

  // This workgroup's item: request r, query tile from token t0, key tiles
  // [tile_begin, tile_cap), and the workspace slot of its partial (-1: the
  // item covers its query tile's keys and writes the rows out).
  // The reference rounding also numbers every item (tile_first + piece,
  // one piece included) for its (max, sum) slots; the tile's pieces are
  // [tile_first, tile_first + npieces).
  int64_t r, q_begin, slot, tile_first, piece, npieces;
  int q_len, ctx, t0, tile_begin, tile_cap;
  if (sc.count > 0) {
    if (wg_item >= sc.count) return;  // uniform over the workgroup
    const uint32_t it = sc.item[wg_item];
    const int k = (int)(it & 0xff);
    const uint32_t tl = sc.tile[k];
    r = (int64_t)(tl & 0xff);
    tile_begin = (int)sc.item_begin[wg_item];
    tile_cap = tile_begin + (int)(it >> 16);
    q_begin = sc.q_begin[k];
    q_len = sc.q_len[k];
    ctx = sc.ctx[k];
    t0 = sc.t0[k];
    npieces = (tl >> 8) & 0xff;
    tile_first = (int64_t)(tl >> 16);
    piece = (int64_t)((it >> 8) & 0xff);
    slot = npieces == 1 ? -1 : tile_first + piece;
  } else {
    // in reverse order: a request's later query tiles see more keys, so the
    // longest items start first and the short ones fill the end of the
    // launch (indices past the call's items exit here, first)
    const PrefillItem pit = prefill_locate(a, (int64_t)(a.grid_items - 1 - wg_item));
    if (pit.r < 0) return;  // uniform over the workgroup
    // (query tile, split) of this item; the loop is wave-uniform (none when
    // every query tile of the request is one piece)
    int qt = 0, split = (int)pit.local, nsplit = 1;
    if ((pit.ctx + pit.q_len + kTileKeys - 1) / kTileKeys <= S) {
      qt = split;
      split = 0;
    } else {
      SplitWalk w;
      w.start(pit.q_len, pit.ctx, tpt, S);
      while (split >= w.nsplit && w.nsplit > 0) {  // nsplit >= 1 for a request with query tokens
        split -= w.nsplit;
        ++qt;
        w.next();
      }
      nsplit = w.nsplit;
    }
    r = pit.r;
    q_begin = pit.q_begin;
    q_len = pit.q_len;
    ctx = pit.ctx;
    t0 = qt * tpt;
    tile_begin = split * S;
    tile_cap = tile_begin + S;
    slot = nsplit == 1 ? -1 : pit.first + pit.local;
    piece = split;
    npieces = nsplit;
    tile_first = pit.first + pit.local - split;
  }
  r = uniform64(r);
  q_begin = uniform64(q_begin);
  slot = uniform64(slot);
  tile_first = uniform64(tile_first);
  piece = uniform64(piece);
  npieces = uniform64(npieces);
  q_len = __builtin_amdgcn_readfirstlane(q_len);
  ctx = __builtin_amdgcn_readfirstlane(ctx);
  t0 = __builtin_amdgcn_readfirstlane(t0);
  tile_begin = __builtin_amdgcn_readfirstlane(tile_begin);
  tile_cap = __builtin_amdgcn_readfirstlane(tile_cap);
  const int t_end = min(t0 + tpt, q_len);
  const int key_end = ctx + t_end;
  if constexpr (kMode == kPrefillStats) {
    if (parts == 2) {
      // the first part takes the first half of the piece's steps (rounded
      // up), the second the rest (none for a one-step piece)
      const int steps = (min(tile_cap, (key_end + kTileKeys - 1) / kTileKeys) - tile_begin + kSub - 1) / kSub;
      const int first_steps = (steps + 1) / 2;
      if (part == 0) {
        tile_cap = tile_begin + first_steps * kSub;
      } else {
        tile_begin += first_steps * kSub;
      }
    }
  }
  const int tile_end = min(tile_cap, (key_end + kTileKeys - 1) / kTileKeys);
  const int last = min(tile_end * kTileKeys, key_end) - 1;  // last key this item reads
  const int last_key0 = (last / kTileKeys) * kTileKeys;     // first key of the tile holding it
  const int32_t* table = a.tables + r * a.table_stride;
  const int tlen = (int)a.table_stride;
  const T* kc = reinterpret_cast<const T*>(a.k_cache) + h * D;
  const T* vc = reinterpret_cast<const T*>(a.v_cache) + h * D;

  // the block-table window first: the first K/V fetch waits for it, the Q
  // rows only the first scores
  TableWindows<kWindows> tc;
  if constexpr (kUniform) {
    const int first_block = (tile_begin * kTileKeys) >> a.geom.bs_shift;
    tc.load(table, tlen, first_block, (last >> a.geom.bs_shift) - first_block + 1);
  }

  // Rows: block nb of this wave = tokens t0 + (wave*kRowBlocks + nb)*(16/G) + row/G, head row%G.
  const int tpb = 16 / a.group;  // tokens per row block
  F qf[kRowBlocks];
  SoftmaxState<D> st[kRowBlocks];
  int q_pos[kRowBlocks];
#pragma unroll
  for (int nb = 0; nb < kRowBlocks; ++nb) {
    const int tq = t0 + (wave * kRowBlocks + nb) * tpb + row / a.group;
    const int qh = h * a.group + row % a.group;
    q_pos[nb] = tq < t_end ? ctx + tq : -1;  // -1: no keys visible (padding row)
    // a padding row reads the tile's last row (no branch around the loads);
    // it has its own MFMA column and is never written
    const int tq_read = min(tq, t_end - 1);
    load_slice<T, D>(qf[nb], reinterpret_cast<const T*>(a.q) + (q_begin + tq_read) * a.q_st + qh * a.q_sh);
    st[nb].init();
  }
  // first and last position of each row block (wave-uniform): steps past
  // the last are fully masked, steps up to the first fully visible
  int block_first[kRowBlocks], block_last[kRowBlocks];
#pragma unroll
  for (int nb = 0; nb < kRowBlocks; ++nb) {
    block_first[nb] = ctx + t0 + (wave * kRowBlocks + nb) * tpb;
    block_last[nb] = min(ctx + t0 + (wave * kRowBlocks + nb + 1) * tpb, key_end) - 1;
  }


  // This wave's DMA ops of the step starting at key0: the K ops then the V
  // ops of the step's tile `wave` (op = wave*kOwnOps + i, the tile's LDS
  // position), so one table lookup serves all of them.  A tile past the
  // item's last key is redirected to the tile that holds it, and rows past
  // it to it (no lane reads a slot the sequence does not own; those keys are
  // masked to p = 0).
  static_assert(kOwnOps == (kFetchV ? 2 : 1) * GT::kOps, "one tile's K (and V) ops per wave");
  // Per-lane element offsets of this wave's ops inside a tile (the same for
  // every tile): the lane's row and its swizzled 16-byte chunk.
  int op_row[kOwnOps], op_row_off[kOwnOps], op_chunk_off[kOwnOps];
#pragma unroll
  for (int i = 0; i < kOwnOps; ++i) {
    const int rr = (i % GT::kOps) * GT::kRowsPerOp + lane / GT::kChunks;
    op_row[i] = rr;
    op_row_off[i] = rr * a.geom.row_elems32;
    op_chunk_off[i] = ((lane % GT::kChunks) ^ GT::swz(rr)) * kEltPerChunk;
  }
  auto issue = [&](int slot, int key0) {
    unsigned char* base = &ring[slot][0] + wave * kOwnOps * kWave * 16;
    const int tkey0 = min(key0 + wave * kTileKeys, last_key0);
    if constexpr (kUniform) {
      // the tile lies in one block: one wave-uniform table lookup, then the
      // lane's row (clamped to the item's last key) and chunk
      const int lb = min(tkey0 >> a.geom.bs_shift, tlen - 1);
      int phys = tc.lookup_forward(lb);
      phys = phys < 0 ? 0 : (phys >= a.geom.num_blocks ? a.geom.num_blocks - 1 : phys);
      const int64_t tile = a.geom.layer_offset +
                           ((int64_t)phys * a.geom.block_size + (tkey0 & (a.geom.block_size - 1))) *
                               a.geom.row_elems;
      const T* kt = kc + tile;
      const T* vt = vc + tile;
      const int row_cap = (last - tkey0) * a.geom.row_elems32;
#pragma unroll
      for (int i = 0; i < kOwnOps; ++i) {
        const int off = min(op_row_off[i], row_cap) + op_chunk_off[i];
        lds_dma16<kPrefillCachePolicy>((i < GT::kOps ? kt : vt) + off, base + i * kWave * 16);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kOwnOps; ++i) {
        const int64_t src = token_offset(a.geom, table, tlen, tkey0 + min(op_row[i], last - tkey0)) + op_chunk_off[i];
        lds_dma16<kPrefillCachePolicy>((i < GT::kOps ? kc : vc) + src, base + i * kWave * 16);
      }
    }
  };

  // Per-lane LDS offsets inside one 16-key tile (K at 0, V at GT::kBytes).
  uint32_t koff[F::kVec];
#pragma unroll
  for (int j = 0; j < F::kVec; ++j) koff[j] = GT::chunk_offset(row, (64 * j + 16 * g) >> 4);
  uint32_t voff[(D / 16) * 4];  // fp32: V^T elements read one by one
  uint32_t vtr[D / 16];         // bf16: transposing reads
#pragma unroll
  for (int c = 0; c < D / 16; ++c) {
    vtr[c] = GT::kBytes + GT::vt_offset(lane, 0, c);
#pragma unroll
    for (int e = 0; e < 4; ++e) voff[4 * c + e] = GT::kBytes + GT::elt_offset(4 * g + e, 0, 16 * c + row);
  }
  constexpr int kTileStride = kOwnOps * kWave * 16;  // K tile + V tile (the stats pass: K only)

  // exp2 multiplier of the scores (see softmax_step)
  const float exp_c = kPow2Scale ? a.scale * kLog2e : kLog2e;

  // Causal boundary or item end inside the step starting at key0: scores of
  // keys a row may not see become -inf (key key0 + 16t + 4g + i is visible
  // iff 16t + i <= lim).  With a false result every key of the step is
  // visible to every row of this wave.
  auto step_full = [&](int key0) { return key0 + kSub * kTileKeys - 1 <= min(block_first[0], last); };
  auto mask_step = [&](v4f (&p)[kRowBlocks][kSub], int key0) {
#pragma unroll
    for (int nb = 0; nb < kRowBlocks; ++nb) {
      const int lim = min(q_pos[nb], last) - (key0 + 4 * g);
#pragma unroll
      for (int t = 0; t < kSub; ++t) {
#pragma unroll
        for (int i = 0; i < 4; ++i) p[nb][t][i] = (t * kTileKeys + i <= lim) ? p[nb][t][i] : kNegInf;
      }
    }
  };

  const int nsteps = (tile_end - tile_begin + kSub - 1) / kSub;
  // steps fetched ahead of the one being consumed; bf16 holds one stage more
  // for the V of the step whose P.V is still to run (see below)
  constexpr int kAhead = Elt<T>::kIsBf16 ? kStages - 2 : kStages - 1;
  static_assert(kAhead >= 1, "at least one step in flight");
  // only steps the item has are fetched
#pragma unroll
  for (int j = 0; j < kAhead; ++j) {
    if (j < nsteps) issue(j, (tile_begin + j * kSub) * kTileKeys);
  }

  // the scale a difference of two (possibly unscaled) scores still takes
  const float score_f = kPow2Scale ? a.scale : 1.f;
  // Exact pass: each row's -m (scaled), l and 1 / l over every piece of its
  // query tile (rows >= the tile's tokens: m = -inf, never written)
  float row_nm[kRowBlocks], row_r[kRowBlocks];
  if constexpr (kMode == kPrefillExact) {
    constexpr int kB = 8;  // pieces per lane group per round trip
#pragma unroll
    for (int nb = 0; nb < kRowBlocks; ++nb) {
      const int64_t rowidx = (wave * kRowBlocks + nb) * 16 + row;
      float m = kNegInf, l = 0.f;
      // the stats pass's parts of the tile's pieces, in order
      const int64_t sparts = a.stats_parts;
      const int64_t nst = npieces * sparts, st0 = tile_first * sparts;
      if (a.ws_ml != nullptr && st0 + nst <= a.ws_ml_slots) {
        for (int64_t p0 = 0; p0 < nst; p0 += 4 * kB) {
          float2 v[kB];
#pragma unroll
          for (int jb = 0; jb < kB; ++jb) {
            const int64_t pc = p0 + 4 * jb + g;
            v[jb] = pc < nst ? *reinterpret_cast<const float2*>(
                                   a.ws_ml + (((st0 + pc) * a.geom.kv_heads + h) * kRows + rowidx) * 2)
                             : make_float2(kNegInf, 0.f);
          }
#pragma unroll
          for (int jb = 0; jb < kB; ++jb) {
            const float mn = score_max(m, v[jb].x);
            if (mn != kNegInf) l = fmaf(l, exp_ref(m - mn), v[jb].y * exp_ref(v[jb].x - mn));  // one explicit fma: with two products the compiler may fuse either
            m = mn;
          }
        }
      }
      const float mm = max_over_groups(m);
      const float ll = sum_over_groups(mm == kNegInf ? 0.f : l * exp_ref(m - mm));
      row_nm[nb] = mm == kNegInf ? 0.f : -mm;
      row_r[nb] = 1.f / ll;
    }
  }

  if constexpr (kMode == kPrefillStats) {
    // K only, one step at a time: the step's scores (the reference's
    // rounding), the row's running maximum and its sum of e^(s - m), each
    // step's 16 exponentials of a row block summed in fp32 (pairwise) and
    // the steps in fp64, rescaled when the maximum moves
    constexpr int kKR = kSub * F::kVec;
    const uint32_t ring0 = lds_off(&ring[0][0]);
    float run_m[kRowBlocks];
    double run_l[kRowBlocks];
#pragma unroll
    for (int nb = 0; nb < kRowBlocks; ++nb) {
      run_m[nb] = kNegInf;
      run_l[nb] = 0.0;
    }
    for (int s0 = 0; s0 < nsteps; s0 += kStages) {
#pragma unroll
      for (int j = 0; j < kStages; ++j) {
        const int s = s0 + j;
        if (s >= nsteps) break;  // uniform over the workgroup
        wait_dma_groups<kOwnOps, kAhead - 1>(min(kAhead - 1, nsteps - 1 - s));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        if (s + kAhead < nsteps) issue((j + kAhead) % kStages, (tile_begin + (s + kAhead) * kSub) * kTileKeys);
        __builtin_amdgcn_sched_barrier(0);
        const int key0 = (tile_begin + s * kSub) * kTileKeys;
        v4u kr[kKR];
        uint32_t kb[F::kVec];
#pragma unroll
        for (int jj = 0; jj < F::kVec; ++jj) kb[jj] = ring0 + j * kStageBytes + koff[jj];
        ring_read_at<kKR, F::kVec, kTileStride>(kr, kb);
#pragma unroll
        for (int jj = 0; jj < kKR; jj += 4) {
          asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(kr[jj]), "+v"(kr[jj + 1]), "+v"(kr[jj + 2]), "+v"(kr[jj + 3]));
        }
        v4f p[kRowBlocks][kSub];
#pragma unroll
        for (int nb = 0; nb < kRowBlocks; ++nb) {
#pragma unroll
          for (int t = 0; t < kSub; ++t) {
            v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int jj = 0; jj < F::kVec; ++jj) {
              acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kr[t * F::kVec + jj]),
                                                            __builtin_bit_cast(bf16x8_t, qf[nb].v[jj]), acc, 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              p[nb][t][i] = kPow2Scale ? round_bf16_in_f32(acc[i]) : scaled_score<T>(acc[i], a.scale);
            }
          }
        }
        if (!step_full(key0)) mask_step(p, key0);
#pragma unroll
        for (int nb = 0; nb < kRowBlocks; ++nb) {
          float lm = kNegInf;
#pragma unroll
          for (int t = 0; t < kSub; ++t) {
            lm = score_max(score_max(lm, score_max(p[nb][t][0], p[nb][t][1])), score_max(p[nb][t][2], p[nb][t][3]));
          }
          const float m_new = score_max(run_m[nb], max_over_groups(lm));
          if (m_new != kNegInf) {
            if (run_m[nb] != m_new) run_l[nb] *= (double)fast_exp2((run_m[nb] - m_new) * score_f * kLog2e);
            // e^(s - m) as 2^(s c - m c), one fma per score (as the decode
            // kernels form their sums)
            const float ec = score_f * kLog2e;
            const float nref = -m_new * ec;
            float e[kSub];
#pragma unroll
            for (int t = 0; t < kSub; ++t) {
              float q4[4];
#pragma unroll
              for (int i = 0; i < 4; ++i) q4[i] = fast_exp2(fmaf(p[nb][t][i], ec, nref));
              e[t] = (q4[0] + q4[1]) + (q4[2] + q4[3]);
            }
            run_l[nb] += (double)((e[0] + e[1]) + (e[2] + e[3]));
          }
          run_m[nb] = m_new;
        }
      }
    }
    // every fetch has been waited for; the piece's (max, sum) per row (max
    // in scaled units; a + b == b + a, so every lane of a row forms the
    // same sum)
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    const int64_t stats_slot = (tile_first + piece) * parts + part;
#pragma unroll
    for (int nb = 0; nb < kRowBlocks; ++nb) {
      double tl = run_l[nb] + __shfl_xor(run_l[nb], 16);
      tl = tl + __shfl_xor(tl, 32);
      const int64_t rowidx = (wave * kRowBlocks + nb) * 16 + row;
      if (g == 0 && a.ws_ml != nullptr && stats_slot < a.ws_ml_slots) {
        const float m = run_m[nb] == kNegInf ? kNegInf : run_m[nb] * score_f;
        *reinterpret_cast<float2*>(a.ws_ml + ((stats_slot * a.geom.kv_heads + h) * kRows + rowidx) * 2) =
            make_float2(m, (float)tl);
      }
    }
    return;
  } else if constexpr (Elt<T>::kIsBf16) {
    // Software-pipelined steps.  Iteration s runs the softmax of step s on
    // scores whose QK MFMAs were issued in iteration s-1.  The P.V MFMAs of
    // step s-1 (its P kept from the previous iteration, its V still in the
    // ring) run beside the rounding of step s, and the QK MFMAs of step s+1
    // beside the exponentials of step s, so both VALU phases of a step have
    // this wave's own MFMAs to overlap with and no MFMA waits on an
    // instruction just before it.  The row sums of P come from an MFMA with
    // an all-ones A operand (the same bf16 P the P.V MFMAs consume), so the
    // softmax has no per-score additions.  LDS reads use immediate offsets
    // from one base address per K vector and per 16-dim V^T chunk.
    constexpr int kKR = kSub * F::kVec;  // K reads per step
    constexpr int kVT = kSub * (D / 16);  // V^T reads per step
    static_assert(kKR % 4 == 0 && kVT % 4 == 0, "reads are waited for in groups of four");
    static_assert(kStages >= kAhead + 2, "a step's V stays in the ring until its P.V has run");
    const uint32_t ring0 = lds_off(&ring[0][0]);
    const bf16x8_t ones = __builtin_bit_cast(bf16x8_t, v4u{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});
    v4f rowsum[kRowBlocks];
#pragma unroll
    for (int nb = 0; nb < kRowBlocks; ++nb) rowsum[nb] = v4f{0.f, 0.f, 0.f, 0.f};
    v4u kr[kKR];
    v2u vt[kVT];
    v4f sacc[kRowBlocks][kSub];

    auto read_k = [&](int slot) {
      const uint32_t sb = ring0 + slot * kStageBytes;
      uint32_t base[F::kVec];
#pragma unroll
      for (int j = 0; j < F::kVec; ++j) base[j] = sb + koff[j];
      ring_read_at<kKR, F::kVec, kTileStride>(kr, base);
    };
    auto read_vt = [&](int slot) {
      const uint32_t sb = ring0 + slot * kStageBytes;
      uint32_t base[D / 16];
#pragma unroll
      for (int c = 0; c < D / 16; ++c) base[c] = sb + vtr[c];
      ring_read_tr_at<kVT, D / 16, kTileStride>(vt, base);
    };
    // every LDS read issued so far has landed; the K (or V^T) operands pass
    // through the asm, so nothing reads them before it and the other set's
    // registers stay free to be reused
    auto wait_k = [&]() {
#pragma unroll
      for (int j = 0; j < kKR; j += 4) {
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(kr[j]), "+v"(kr[j + 1]), "+v"(kr[j + 2]), "+v"(kr[j + 3]));
      }
    };
    auto wait_vt = [&]() {
#pragma unroll
      for (int j = 0; j < kVT; j += 4) {
        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(vt[j]), "+v"(vt[j + 1]), "+v"(vt[j + 2]), "+v"(vt[j + 3]));
      }
    };
    auto qk = [&]() {
#pragma unroll
      for (int nb = 0; nb < kRowBlocks; ++nb) {
#pragma unroll
        for (int t = 0; t < kSub; ++t) {
          v4f acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int j = 0; j < F::kVec; ++j) {
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, kr[t * F::kVec + j]),
                                                          __builtin_bit_cast(bf16x8_t, qf[nb].v[j]), acc, 0, 0, 0);
          }
          sacc[nb][t] = acc;
        }
      }
    };

    // prologue: step 0 landed, its scores issued
    wait_dma_groups<kOwnOps, kAhead - 1>(min(kAhead - 1, nsteps - 1));
    __builtin_amdgcn_s_barrier();
    read_k(0);
    wait_k();
    qk();

    // A row's reference point moves when one of its scores is more than
    // kRescaleLog2 (log2 units) above it, i.e. more than grow_thr in score
    // units; nref = -m * exp_c is kept with it (0 while m = -inf, so that a
    // row with nothing unmasked yet gets exact zeros, not NaN).
    const float grow_thr = kRescaleLog2 / exp_c;
    float nref[kRowBlocks];
#pragma unroll
    for (int nb = 0; nb < kRowBlocks; ++nb) nref[nb] = 0.f;

    // O^T += V^T . P^T and the row sums for the P of one step (pp) and its
    // V^T operands (vt), two 16-key tiles per MFMA
    auto pv = [&](const bf16x8_t (&pp)[kRowBlocks][kSub / 2]) {
#pragma unroll
      for (int t = 0; t < kSub; t += 2) {
#pragma unroll
        for (int nb = 0; nb < kRowBlocks; ++nb) {
#pragma unroll
          for (int c = 0; c < D / 16; ++c) {
            const bf16x8_t vv = join_bf16x4(__builtin_bit_cast(v4s, vt[t * (D / 16) + c]),
                                            __builtin_bit_cast(v4s, vt[(t + 1) * (D / 16) + c]));
            st[nb].o[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vv, pp[nb][t / 2], st[nb].o[c], 0, 0, 0);
          }
          if constexpr (kMode == kPrefillOnline) {
            rowsum[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pp[nb][t / 2], rowsum[nb], 0, 0, 0);
          }
        }
      }
    };
    bf16x8_t pp_prev[kRowBlocks][kSub / 2];  // P of the step whose P.V is still to run

    // Iteration s in ring stage `slot`.  more: a step s+1 exists (its scores
    // are issued here); prev: a step s-1 exists (its P.V runs here).  Both
    // are literals at every call site, so each call is straight-line code.
    auto step = [&](int slot, int s, bool more, bool prev) {
      set_wave_priority(nsteps - s);  // the workgroup with more steps left goes first
      if (more) {
        // step s+1 has landed for every wave (this wave's ops: at most
        // those of the steps issued after it remain), and every wave has
        // finished iteration s-1, so the stage the next fetch reuses (last
        // read for step s-2's V) is free
        wait_dma_groups<kOwnOps, kAhead - 2>(min(kAhead - 2, nsteps - 2 - s));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        if (s + kAhead < nsteps) issue((slot + kAhead) % kStages, (tile_begin + (s + kAhead) * kSub) * kTileKeys);
      }
      if (prev) read_vt((slot + kStages - 1) % kStages);
      __builtin_amdgcn_sched_barrier(0);

      // softmax of step s: scores in the reference's rounding (the q.k sum
      // rounded to bf16, times the scale, rounded again; the second rounding
      // is exact and the scale moves into exp_c when the scale is a power of
      // two)
      const int key0 = (tile_begin + s * kSub) * kTileKeys;
      v4f p[kRowBlocks][kSub];
#pragma unroll
      for (int nb = 0; nb < kRowBlocks; ++nb) {
#pragma unroll
        for (int t = 0; t < kSub; ++t) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            p[nb][t][i] = kPow2Scale ? round_bf16_in_f32(sacc[nb][t][i]) : scaled_score<T>(sacc[nb][t][i], a.scale);
          }
        }
      }
      if (prev) {
        wait_vt();
        pv(pp_prev);  // step s-1, against the reference points its P was formed with
      }
      // K of step s+1 (landed: waited for above), read only now so its
      // registers are not held across the P.V of step s-1
      if (more) read_k((slot + 1) % kStages);
      if (!step_full(key0)) mask_step(p, key0);
      if constexpr (kMode == kPrefillExact) {
        // P = e^(s - m) / l with the row's final (m, l): s - m exact (the
        // unscaled score times a power-of-two scale, minus m, rounds once,
        // as the reference's input - max), then 2^((s - m) log2 e) and a
        // product with 1 / l.  That is a few fp32 ulps from the reference's
        // exp and division (exp_ref / div_ref would halve the gap at
        // 1.3-1.5x the call time); in the 16 x 256 serving lockstep both
        // forms agree with the reference path as well as its fp32-product
        // variant does (top-1 95.2% either way, median logit error 0.086).
#pragma unroll
        for (int t = 0; t < kSub; t += 2) {
#pragma unroll
          for (int nb = 0; nb < kRowBlocks; ++nb) {
#pragma unroll
            for (int u = t; u < t + 2; ++u) {
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const float x = kPow2Scale ? fmaf(p[nb][u][i], a.scale, row_nm[nb]) : p[nb][u][i] + row_nm[nb];
                p[nb][u][i] = fast_exp2(x * kLog2e) * row_r[nb];
              }
            }
            pp_prev[nb][t / 2] = join_bf16x4(pack_bf16x4(p[nb][t][0], p[nb][t][1], p[nb][t][2], p[nb][t][3]),
                                             pack_bf16x4(p[nb][t + 1][0], p[nb][t + 1][1], p[nb][t + 1][2],
                                                         p[nb][t + 1][3]));
          }
        }
        if (more) {
          wait_k();
          qk();  // scores of step s+1
        }
        return;
      }
      // each lane tests its own 16 scores of a row; only when one of them
      // moves the row's reference point is the row maximum formed across
      // the lane groups (see softmax_step).  m = -inf gives +inf (a finite
      // score grows it), a fully masked lane gives -inf or NaN (no growth).
      float lmax[kRowBlocks];
      bool grow = false;
#pragma unroll
      for (int nb = 0; nb < kRowBlocks; ++nb) {
        float m0 = score_max(score_max(p[nb][0][0], p[nb][0][1]), p[nb][0][2]);
        float m1 = score_max(score_max(p[nb][0][3], p[nb][1][0]), p[nb][1][1]);
        m0 = score_max(score_max(m0, p[nb][1][2]), p[nb][1][3]);
        m1 = score_max(score_max(m1, p[nb][2][0]), p[nb][2][1]);
        m0 = score_max(score_max(m0, p[nb][2][2]), p[nb][2][3]);
        m1 = score_max(score_max(m1, p[nb][3][0]), p[nb][3][1]);
        m0 = score_max(score_max(m0, p[nb][3][2]), p[nb][3][3]);
        lmax[nb] = score_max(m0, m1);
        grow |= lmax[nb] - st[nb].m > grow_thr;
      }
      if (__ballot(grow)) {
        // O and the sums hold every step up to s-1 (relative to the old
        // reference points); they move to the new ones together
#pragma unroll
        for (int nb = 0; nb < kRowBlocks; ++nb) {
          const float m_new = score_max(st[nb].m, max_over_groups(lmax[nb]));
          // alpha = 0 for a row without a reference yet (its O and sum are 0)
          const float alpha = st[nb].m == kNegInf ? 0.f : fast_exp2((st[nb].m - m_new) * exp_c);
          rowsum[nb] *= alpha;
#pragma unroll
          for (int c = 0; c < D / 16; ++c) st[nb].o[c] *= alpha;
          st[nb].m = m_new;
          nref[nb] = m_new == kNegInf ? 0.f : -m_new * exp_c;
        }
      }
#pragma unroll
      for (int t = 0; t < kSub; t += 2) {
#pragma unroll
        for (int nb = 0; nb < kRowBlocks; ++nb) {
#pragma unroll
          for (int u = t; u < t + 2; ++u) {
#pragma unroll
            for (int i = 0; i < 4; ++i) p[nb][u][i] = fast_exp2(fmaf(p[nb][u][i], exp_c, nref[nb]));
          }
          pp_prev[nb][t / 2] = join_bf16x4(pack_bf16x4(p[nb][t][0], p[nb][t][1], p[nb][t][2], p[nb][t][3]),
                                           pack_bf16x4(p[nb][t + 1][0], p[nb][t + 1][1], p[nb][t + 1][2],
                                                       p[nb][t + 1][3]));
        }
      }
      if (more) {
        wait_k();
        qk();  // scores of step s+1
      }
    };

    // Step 0 has no predecessor and the last step no successor (its ring
    // stage is known only at run time: the reads take it from their base
    // address); the steps between run unrolled over the ring's stages.
    if (nsteps > 1) step(0, 0, true, false);
    for (int s0 = 1; s0 < nsteps - 1; s0 += kStages) {
#pragma unroll
      for (int j = 0; j < kStages; ++j) {
        const int s = s0 + j;
        if (s >= nsteps - 1) break;  // uniform over the workgroup
        step((1 + j) % kStages, s, true, true);
      }
    }
    if (nsteps == 1) {
      step(0, 0, false, false);
    } else if (nsteps > 1) {
      step((nsteps - 1) % kStages, nsteps - 1, false, true);
    }
    // P.V of the last step
    if (nsteps > 0) {
      read_vt((nsteps - 1) % kStages);
      wait_vt();
      pv(pp_prev);
    }
#pragma unroll
    for (int nb = 0; nb < kRowBlocks; ++nb) st[nb].lsum = kMode == kPrefillExact ? 1.f : rowsum[nb][0];
  } else {
    auto consume = [&](int slot, int key0) {
      const unsigned char* stage = &ring[slot][0];
      v4f p[kRowBlocks][kSub];
      F kf[kSub];
#pragma unroll
      for (int t = 0; t < kSub; ++t) {
#pragma unroll
        for (int j = 0; j < F::kVec; ++j) {
          kf[t].v[j] = *reinterpret_cast<const uint4*>(stage + t * kTileStride + koff[j]);
        }
      }
#pragma unroll
      for (int nb = 0; nb < kRowBlocks; ++nb) {
#pragma unroll
        for (int t = 0; t < kSub; ++t) {
          p[nb][t] = qk_mfma<T, D>(kf[t], qf[nb]);
#pragma unroll
          for (int i = 0; i < 4; ++i) p[nb][t][i] = scaled_score<T>(p[nb][t][i], a.scale);
        }
      }
      if (!step_full(key0)) mask_step(p, key0);
      softmax_step<D, kRowBlocks, kSub>(st, p, exp_c);
#pragma unroll
      for (int t = 0; t < kSub; ++t) {
#pragma unroll
        for (int c = 0; c < D / 16; ++c) {
          float vv[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) vv[j] = *reinterpret_cast<const float*>(stage + t * kTileStride + voff[4 * c + j]);
#pragma unroll
          for (int nb = 0; nb < kRowBlocks; ++nb) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              st[nb].o[c] = __builtin_amdgcn_mfma_f32_16x16x4f32(vv[j], p[nb][t][j], st[nb].o[c], 0, 0, 0);
            }
          }
        }
      }
    };
    for (int s0 = 0; s0 < nsteps; s0 += kStages) {
#pragma unroll
      for (int j = 0; j < kStages; ++j) {
        const int s = s0 + j;
        if (s >= nsteps) break;  // uniform over the workgroup
        // this wave's ops for step s are done once at most the ops of the
        // steps issued after it (min(kAhead - 1, nsteps - 1 - s)) are
        // outstanding; the barrier extends that to every wave and guarantees
        // that every wave has finished reading step s-1, whose stage the next
        // fetch reuses
        wait_dma_groups<kOwnOps, kAhead - 1>(min(kAhead - 1, nsteps - 1 - s));
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
        if (s + kAhead < nsteps) issue((j + kAhead) % kStages, (tile_begin + (s + kAhead) * kSub) * kTileKeys);
        __builtin_amdgcn_sched_barrier(0);
        consume(j, (tile_begin + s * kSub) * kTileKeys);
      }
    }
#pragma unroll
    for (int nb = 0; nb < kRowBlocks; ++nb) st[nb].lsum = sum_over_groups(st[nb].lsum);
  }
  // every fetch has been waited for (the last step's wait is vmcnt(0))
  __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));

#pragma unroll
  for (int nb = 0; nb < kRowBlocks; ++nb) {
    const float lsum = st[nb].lsum;
    const int tq = t0 + (wave * kRowBlocks + nb) * tpb + row / a.group;
    if (tq >= t_end) continue;
    const int qh = h * a.group + row % a.group;
    if (slot < 0) {
      const float inv = 1.f / lsum;
      T* dst = reinterpret_cast<T*>(a.out) + (q_begin + tq) * a.o_st + qh * a.o_sh + 4 * g;
#pragma unroll
      for (int c = 0; c < D / 16; ++c) {
        store4<T>(dst + 16 * c, st[nb].o[c][0] * inv, st[nb].o[c][1] * inv, st[nb].o[c][2] * inv,
                  st[nb].o[c][3] * inv);
      }
    } else if (a.ws_o != nullptr && slot < a.ws_items) {
      const int64_t wrow = (slot * a.geom.kv_heads + h) * kRows + (wave * kRowBlocks + nb) * 16 + row;
      float* dst = a.ws_o + wrow * D + 4 * g;
#pragma unroll
      // streaming stores: the partials drain to memory while other items
      // still run, instead of in the L2 writeback at the end of the kernel
      // (mixed chunked-prefill step: 26.4 -> 25.6 us per call)
      for (int c = 0; c < D / 16; ++c) {
        __builtin_nontemporal_store(st[nb].o[c], reinterpret_cast<v4f*>(dst + 16 * c));
      }
      // the merge expects the maximum of the scaled scores (the exact pass
      // leaves the slots alone: other pieces of its tile may still be
      // reading their stats there, and the summing merge needs none)
      const float m = kPow2Scale ? st[nb].m * a.scale : st[nb].m;
      if (kMode == kPrefillOnline && g == 0) {
        __builtin_nontemporal_store(m, a.ws_ml + wrow * 2);
        __builtin_nontemporal_store(lsum, a.ws_ml + wrow * 2 + 1);
      }
    }
  }
}

// Merge of split prefill rows: a workgroup takes 32 rows (blockIdx.z) of a
// split query tile (blockIdx.x: merge job j, or without jobs the x-th query
// tile of the call, located on the device), for one KV head (blockIdx.y);
// wave w takes 4 of those rows, lane l the 4-dim chunk l%16 (and l%16 + 16,
// ... for larger head_dim) of row l/16.  Every split's loads of a batch of
// up to kBatch splits are issued before any is used, so the usual merge is
// one memory round trip; batches combine through a running maximum per row
// (exact log-sum-exp weights, splits in order).  kBatch is the launch's
// largest split count rounded up to 4, 8 or 16: the batch's registers set
// how many merge workgroups a CU holds (234 VGPRs for 21 splits at head_dim
// 64 allow one, so the 384 to 544 workgroups of a serving step's prefill
// merge ran in two or three rounds: 9-12 us against 4-5 us in one).
constexpr int kPrefillMergeWaves = 8;
constexpr int kPrefillMergeRows = kPrefillMergeWaves * 4;

// Sum of prefill_items_of over the sequences before r (wave-uniform).
__device__ __forceinline__ int64_t prefill_items_before(const PrefillArgs& a, int64_t r) {
  int64_t n = 0;
  for (int64_t b = lane_id(); b < r; b += kWave) n += prefill_items_of(a, b);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) n += __shfl_xor(n, off);
  return uniform64(n);
}

// The split query tiles of a call, listed on the host from its exact plan
// and passed by value as a kernel argument: job j = {first item, first
// packed query row, split count, token count} of the j-th split tile.
constexpr int kMaxMergeJobs = 128;

struct PrefillMergeJobs {
  int32_t count;  // 0: locate the tiles on the device instead
  int32_t first_item[kMaxMergeJobs];
  int32_t row0[kMaxMergeJobs];
  int32_t nsplit_tokens[kMaxMergeJobs];  // nsplit << 16 | tokens
};

// kSum: partials of the reference rounding (shares of the normalised
// output): summed in split order, no weights, rounded once.
template <typename T, int D, int kRowBlocks, int kBatch, bool kSum>
__global__ __launch_bounds__(kPrefillMergeWaves* kWave) void prefill_merge_kernel(PrefillArgs a,
                                                                                 PrefillMergeJobs jobs) {
  constexpr int kRows = prefill_rows_per_item<kRowBlocks>();
  constexpr int kChunkPasses = D / 64;  // 4-dim chunks per lane
  static_assert(kBatch >= 1, "splits per round trip");
  const int tpt = a.tokens_per_tile;
  // (query tile, KV head, row group) of this workgroup, head-major over the
  // XCDs like the prefill items whose partials it reads
  constexpr int kGroups = kRows / kPrefillMergeRows;
  const int64_t logical = xcd_logical(blockIdx.x, (int64_t)a.merge_tiles * a.geom.kv_heads * kGroups);
  const int zg = (int)(logical % kGroups);
  const int tile = (int)((logical / kGroups) % a.merge_tiles);
  const int h = (int)(logical / kGroups / a.merge_tiles);
  int64_t first, row0;
  int nsplit, tokens;
  if (jobs.count > 0) {
    const int j = tile;
    first = jobs.first_item[j];
    row0 = jobs.row0[j];
    nsplit = jobs.nsplit_tokens[j] >> 16;
    tokens = jobs.nsplit_tokens[j] & 0xffff;
  } else {
    const int S = a.tiles_per_split;
    int64_t r, qt64, first_q, count_q;
    locate_item((int64_t)tile, a.num_seqs,
                [&](int64_t b) { return (a.cu_seqlens[b + 1] - a.cu_seqlens[b] + tpt - 1) / tpt; }, &r, &qt64,
                &first_q, &count_q);
    if (r < 0) return;  // uniform over the workgroup
    const int qt = (int)qt64;
    const int64_t q_begin = a.cu_seqlens[r];
    const int q_len = (int)(a.cu_seqlens[r + 1] - q_begin);
    const int ctx = a.context_lens[r];
    nsplit = (prefill_key_tiles(ctx, q_len, tpt, qt) + S - 1) / S;
    if (nsplit <= 1) return;  // the prefill kernel wrote these rows
    first = prefill_items_before(a, r) + prefill_items_upto(q_len, ctx, tpt, S, qt);  // the tile's first item
    row0 = q_begin + qt * tpt;
    tokens = min(tpt, q_len - qt * tpt);
  }
  if (first + nsplit > a.ws_items) return;
  const int lane = lane_id();
  const int wave = (int)(threadIdx.x / kWave);
  const int chunk = lane & 15;
  const int rr = zg * kPrefillMergeRows + wave * 4 + (lane >> 4);  // row within the item
  const int tpb = 16 / a.group;
  const int tq = (rr / 16) * tpb + (rr % 16) / a.group;  // token within the tile
  const int64_t split_stride = (int64_t)a.geom.kv_heads * kRows;  // rows between consecutive items
  // split s of this row: the uniform base of slot (first + s, h) plus a
  // lane offset shared by every split, so each load needs no address
  // registers of its own (scalar base, 32-bit vector offset)
  const int64_t row0_first = (first * a.geom.kv_heads + h) * kRows;
  const float* o_first = a.ws_o + row0_first * D;
  const float* ml_first = a.ws_ml + row0_first * 2;
  const uint32_t o_lane = (uint32_t)(rr * D + 4 * chunk);
  const uint32_t ml_lane = (uint32_t)(rr * 2);

  float run_max = kNegInf, denom = 0.f;
  float4 acc[kChunkPasses];
#pragma unroll
  for (int c = 0; c < kChunkPasses; ++c) acc[c] = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int s0 = 0; s0 < nsplit; s0 += kBatch) {
    float4 v[kBatch][kChunkPasses];
    float2 ml[kBatch];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const bool in = s0 + b < nsplit;
      const int64_t split_row = (int64_t)(s0 + b) * split_stride;  // uniform
      const float* ob = o_first + split_row * D;
      if constexpr (!kSum) {
        ml[b] = in ? *reinterpret_cast<const float2*>(ml_first + split_row * 2 + ml_lane) : make_float2(kNegInf, 0.f);
      }
#pragma unroll
      for (int c = 0; c < kChunkPasses; ++c) {
        v[b][c] = in ? *reinterpret_cast<const float4*>(ob + o_lane + 64 * c) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    if constexpr (kSum) {
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
#pragma unroll
        for (int c = 0; c < kChunkPasses; ++c) {
          acc[c].x += v[b][c].x;
          acc[c].y += v[b][c].y;
          acc[c].z += v[b][c].z;
          acc[c].w += v[b][c].w;
        }
      }
      continue;
    }
    float bmax = ml[0].x;
#pragma unroll
    for (int b = 1; b < kBatch; ++b) bmax = fmaxf(bmax, ml[b].x);
    const float new_max = fmaxf(run_max, bmax);
    const float keep = run_max == kNegInf ? 0.f : exp2f((run_max - new_max) * kLog2e);
    denom *= keep;
#pragma unroll
    for (int c = 0; c < kChunkPasses; ++c) {
      acc[c].x *= keep;
      acc[c].y *= keep;
      acc[c].z *= keep;
      acc[c].w *= keep;
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const float w = ml[b].x == kNegInf ? 0.f : exp2f((ml[b].x - new_max) * kLog2e);
      denom += w * ml[b].y;
#pragma unroll
      for (int c = 0; c < kChunkPasses; ++c) {
        acc[c].x += w * v[b][c].x;
        acc[c].y += w * v[b][c].y;
        acc[c].z += w * v[b][c].z;
        acc[c].w += w * v[b][c].w;
      }
    }
    run_max = new_max;
  }
  if (rr >= kRows || tq >= tokens) return;
  const int qh = h * a.group + (rr % 16) % a.group;
  const float inv = kSum ? 1.f : 1.f / denom;
  T* dst = reinterpret_cast<T*>(a.out) + (row0 + tq) * a.o_st + qh * a.o_sh;
#pragma unroll
  for (int c = 0; c < kChunkPasses; ++c) {
    store4<T>(dst + 4 * (chunk + 16 * c), acc[c].x * inv, acc[c].y * inv, acc[c].z * inv, acc[c].w * inv);
  }
}

// Work decomposition of a prefill call: query tiles of tokens_per_tile
// tokens, each split into items of at most tiles_per_split key tiles.  With
// host copies of the lengths the split length fills the GPU's resident
// workgroup slots about once and the grid is exact; without them an upper
// bound on the total work gives about kPrefillTargetItems workgroups.
constexpr int64_t kPrefillTargetItems = 2048;
constexpr int64_t kPrefillMinTilesPerSplit = 8;
// A piece of L >= 2 tiles spans at most L blocks of 16 keys or more, so its
// lookups stay in the kernel's block-table windows.
constexpr int64_t kPrefillMaxTilesPerSplit = kTableWindow * kPrefillTableWindows;

// A query tile of a host-planned prefill call (tiles in request order) and
// its pieces' workspace slots [first, first + pieces).
struct PrefillTile {
  int64_t r;       // request
  int64_t qt;      // query tile within the request
  int64_t ktiles;  // 16-key tiles it sees
  int64_t pieces;
  int64_t first;
};

// One work item: key tiles [begin, begin + len) of query tile `tile`, its
// `piece`-th piece.
struct PrefillPiece {
  int32_t tile, piece, begin, len;
};

struct PrefillPlan {
  int row_blocks = 2;  // MFMA row blocks per wave
  int tokens_per_tile = 64;
  int64_t tps = kPrefillMaxTilesPerSplit;  // piece length of the device-located plan
  int64_t items = 0;   // prefill grid.x per KV head: the item count (exact from host metadata, else a bound)
  int64_t qtiles = 0;  // merge grid.x: the query-tile count (exact, else a bound)
  int64_t rows = 0;    // rows per item
  bool split = false;  // some query tile is split over several items
  int64_t max_split = 0;  // items of the most-split query tile (a bound without host metadata)
  bool long_pieces = false;  // some piece spans more than one block-table window (kTableWindow tiles)
  // host metadata: the query tiles and the items in dispatch order
  std::vector<PrefillTile> tiles;
  std::vector<PrefillPiece> order;
};

// Workgroups a prefill call aims for with host metadata when its pieces are
// uniform: the split length is chosen so the items fill the GPU about once
// (two workgroups fit a CU at head_dim 64; 1.5 per CU measured fastest).
inline int64_t prefill_slots() { return 3 * device_cus() / 2; }

// Key tiles visible to query tile qt of a request with n query tokens after
// ctx cached ones (host side of prefill_key_tiles).
int64_t host_key_tiles(int64_t ctx, int64_t n, int64_t tpt, int64_t qt) {
  const int64_t t_end = (qt + 1) * tpt < n ? (qt + 1) * tpt : n;
  return cdiv(ctx + t_end, (int64_t)kTileKeys);
}

// Balanced pieces for a call whose KV heads each fill one XCD (kv_heads ==
// kXcds, the grid is head-major over the XCDs): every query tile is cut into
// pieces of about half a CU's share of the head's 64-key steps, and the
// pieces are ordered so that the dispatcher, which places the k-th and the
// (k + CUs)-th workgroup of an XCD on one CU, pairs the smallest of the
// large pieces with the largest of the small ones.  False (uniform pieces
// instead) when the call is too small to fill the XCD twice or its pieces
// would not fit the kernel-argument tables.
bool plan_balanced(PrefillPlan& p, int64_t kv_heads) {
  const int64_t ncu = device_cus() / kXcds;
  if (kv_heads != kXcds || ncu < 2 || p.tiles.size() > (size_t)kMaxSchedTiles) return false;
  // only plans the item table can hold: a device-located fallback would cut
  // the tiles into uniform pieces that the balanced merge jobs do not match
  for (const PrefillTile& t : p.tiles) {
    if (t.r > 255) return false;
  }
  const int64_t slots = 2 * ncu;
  int64_t total = 0;
  for (const PrefillTile& t : p.tiles) total += cdiv(t.ktiles, (int64_t)kPrefillStepTiles);
  if (total < slots) return false;
  double half = (double)total / (double)slots;  // steps per piece
  std::vector<int64_t> n(p.tiles.size());
  for (int attempt = 0;; ++attempt) {
    int64_t count = 0;
    for (size_t i = 0; i < p.tiles.size(); ++i) {
      const int64_t steps = cdiv(p.tiles[i].ktiles, (int64_t)kPrefillStepTiles);
      int64_t k = (int64_t)std::llround((double)steps / half);
      const int64_t min_k = cdiv(p.tiles[i].ktiles, kPrefillMaxTilesPerSplit);
      k = k < min_k ? min_k : (k > steps ? steps : k);
      n[i] = k < 1 ? 1 : k;
      count += n[i];
    }
    if (count <= slots) break;
    if (attempt == 64) return false;
    half *= 1.05;
  }
  std::vector<PrefillPiece> pieces;
  int64_t first = 0, splits = 0;
  for (size_t i = 0; i < p.tiles.size(); ++i) {
    PrefillTile& t = p.tiles[i];
    const int64_t steps = cdiv(t.ktiles, (int64_t)kPrefillStepTiles);
    t.pieces = n[i];
    t.first = first;
    first += n[i];
    splits += n[i] > 1;
    int64_t done = 0;  // steps before this piece
    for (int64_t j = 0; j < n[i]; ++j) {
      const int64_t size = steps / n[i] + (j < steps % n[i] ? 1 : 0);
      const int64_t begin = done * kPrefillStepTiles;
      const int64_t len = std::min(size * kPrefillStepTiles, t.ktiles - begin);
      if (begin > 0xffff || len > kPrefillMaxTilesPerSplit) return false;
      pieces.push_back(PrefillPiece{(int32_t)i, (int32_t)j, (int32_t)begin, (int32_t)len});
      done += size;
    }
  }
  if (pieces.size() > (size_t)kMaxSchedItems || splits > kMaxMergeJobs) return false;
  p.max_split = *std::max_element(n.begin(), n.end());
  // the ncu largest in ascending order, then the rest in descending order:
  // dispatch position k < ncu and k + ncu share a CU
  std::vector<PrefillPiece> by_size(pieces);
  std::stable_sort(by_size.begin(), by_size.end(),
                   [](const PrefillPiece& x, const PrefillPiece& y) { return x.len > y.len; });
  const size_t big = std::min((size_t)ncu, by_size.size());
  p.order.assign(by_size.rbegin() + (by_size.size() - big), by_size.rend());
  p.order.insert(p.order.end(), by_size.begin() + big, by_size.end());
  p.items = (int64_t)pieces.size();
  p.split = splits > 0;
  for (const PrefillPiece& q : pieces) p.long_pieces |= q.len > kTableWindow;
  return true;
}

// host_cu / host_ctx: optional host copies of cu_seqlens / context_lens,
// already validated by the caller; without them the plan uses bounds.
PrefillPlan plan_prefill(int64_t group, int64_t kv_heads, int64_t num_seqs, int64_t total_tokens,
                         int64_t max_seq_len, const int64_t* host_cu, const int32_t* host_ctx) {
  PrefillPlan p;
  static const int forced_rb = env_int("NIE_PREFILL_ROW_BLOCKS");
  if (forced_rb == 1 || forced_rb == 2) p.row_blocks = forced_rb;
  p.tokens_per_tile = kPrefillWaves * p.row_blocks * (int)(16 / group);
  p.rows = kPrefillWaves * p.row_blocks * 16;
  const int64_t tpt = p.tokens_per_tile;
  static const int64_t forced = env_int("NIE_PREFILL_TILES_PER_SPLIT");
  auto clamp_tps = [&](int64_t tps) {
    if (forced > 0) tps = forced;
    tps = tps < kPrefillMinTilesPerSplit ? kPrefillMinTilesPerSplit : tps;
    tps = tps > kPrefillMaxTilesPerSplit ? kPrefillMaxTilesPerSplit : tps;
    return cdiv(tps, (int64_t)kPrefillStepTiles) * kPrefillStepTiles;  // whole key steps
  };
  if (host_cu != nullptr && host_ctx != nullptr) {
    int64_t work = 0;
    for (int64_t r = 0; r < num_seqs; ++r) {
      const int64_t n = host_cu[r + 1] - host_cu[r];
      for (int64_t qt = 0; qt < cdiv(n, tpt); ++qt) {
        const int64_t kt = host_key_tiles(host_ctx[r], n, tpt, qt);
        p.tiles.push_back(PrefillTile{r, qt, kt, 0, 0});
        work += kt;
      }
    }
    p.qtiles = (int64_t)p.tiles.size();
    static const int balanced_off = env_int("NIE_PREFILL_UNIFORM");
    if (forced <= 0 && balanced_off <= 0 && plan_balanced(p, kv_heads)) return p;
    // uniform pieces of tps tiles, in request order
    p.tps = clamp_tps(cdiv(work * kv_heads, prefill_slots()));
    p.order.clear();
    int64_t first = 0;
    for (size_t i = 0; i < p.tiles.size(); ++i) {
      PrefillTile& t = p.tiles[i];
      t.pieces = cdiv(t.ktiles, p.tps);
      t.first = first;
      first += t.pieces;
      p.split |= t.pieces > 1;
      p.max_split = std::max(p.max_split, t.pieces);
      for (int64_t j = 0; j < t.pieces; ++j) {
        const int64_t begin = j * p.tps;
        p.order.push_back(PrefillPiece{(int32_t)i, (int32_t)j, (int32_t)begin,
                                       (int32_t)std::min(p.tps, t.ktiles - begin)});
      }
    }
    p.items = first;
    for (const PrefillPiece& q : p.order) p.long_pieces |= q.len > kTableWindow;
    return p;
  }
  const int64_t qtiles = total_tokens / tpt + num_seqs;  // >= sum_r ceil(len_r / tpt)
  const int64_t ktiles = cdiv(max_seq_len, (int64_t)kTileKeys);
  const int64_t work = qtiles * ktiles;                  // >= key tiles over all query tiles
  p.tps = clamp_tps(cdiv(work * kv_heads, kPrefillTargetItems));
  p.items = work / p.tps + qtiles + 1;  // sum ceil(n / tps) <= sum n / tps + count
  p.qtiles = qtiles;
  p.split = ktiles > p.tps;
  p.max_split = cdiv(ktiles, p.tps);
  p.long_pieces = std::min(p.tps, ktiles) > kTableWindow;
  return p;
}

// The split query tiles of a host-planned call as merge jobs (count 0 when
// there are more than kMaxMergeJobs: the merge then locates them itself,
// which needs the uniform pieces of the device-located plan).
void fill_merge_jobs(const PrefillPlan& p, int64_t num_seqs, const int64_t* host_cu, const int32_t* host_ctx,
                     PrefillMergeJobs* jobs) {
  (void)num_seqs;
  (void)host_ctx;
  jobs->count = 0;
  if (host_cu == nullptr || p.tiles.empty()) return;
  const int64_t tpt = p.tokens_per_tile;
  int n = 0;
  for (const PrefillTile& t : p.tiles) {
    if (t.pieces <= 1) continue;
    const int64_t len = host_cu[t.r + 1] - host_cu[t.r];
    const int64_t row0 = host_cu[t.r] + t.qt * tpt;
    if (n == kMaxMergeJobs || t.first > 0x7fffffffLL || row0 > 0x7fffffffLL || t.pieces > 0x7fff) {
      jobs->count = 0;
      return;
    }
    jobs->first_item[n] = (int32_t)t.first;
    jobs->row0[n] = (int32_t)row0;
    const int64_t tokens = len - t.qt * tpt < tpt ? len - t.qt * tpt : tpt;
    jobs->nsplit_tokens[n] = (int32_t)((t.pieces << 16) | tokens);
    ++n;
  }
  jobs->count = n;
}

// The item table of a host-planned call (see PrefillSchedule), in the plan's
// dispatch order.  False when the call has more query tiles or items than
// the table holds (the workgroups then locate their items, which needs the
// uniform pieces of the device-located plan).
bool build_prefill_schedule(const PrefillPlan& p, int64_t num_seqs, const int64_t* host_cu,
                            const int32_t* host_ctx, PrefillSchedule* sc) {
  (void)num_seqs;
  sc->count = 0;
  if (p.tiles.empty() || p.tiles.size() > (size_t)kMaxSchedTiles || p.order.size() > (size_t)kMaxSchedItems ||
      (int64_t)p.order.size() != p.items) {
    return false;
  }
  const int64_t tpt = p.tokens_per_tile;
  for (size_t k = 0; k < p.tiles.size(); ++k) {
    const PrefillTile& t = p.tiles[k];
    const int64_t n = host_cu[t.r + 1] - host_cu[t.r];
    if (t.r > 255 || t.pieces > 255 || t.first > 0xffff || host_cu[t.r] > 0x7fffffffLL || n > 0x7fffffffLL) {
      return false;
    }
    sc->tile[k] = (uint32_t)t.r | (uint32_t)t.pieces << 8 | (uint32_t)t.first << 16;
    sc->q_begin[k] = (int32_t)host_cu[t.r];
    sc->q_len[k] = (int32_t)n;
    sc->ctx[k] = host_ctx[t.r];
    sc->t0[k] = (int32_t)(t.qt * tpt);
  }
  for (size_t i = 0; i < p.order.size(); ++i) {
    const PrefillPiece& q = p.order[i];
    if (q.tile > 255 || q.piece > 255 || q.len > 0xffff || q.begin < 0) return false;
    sc->item[i] = (uint32_t)q.tile | (uint32_t)q.piece << 8 | (uint32_t)q.len << 16;
    sc->item_begin[i] = (uint32_t)q.begin;
  }
  sc->count = (int32_t)p.order.size();
  return true;
}

// Checks host copies of cu_seqlens / context_lens against the call's sizes.
bool host_metadata_ok(const int64_t* host_cu, const int32_t* host_ctx, int64_t num_seqs, int64_t total_tokens,
                      int64_t max_query_len, int64_t max_seq_len) {
  if (host_cu[0] != 0 || host_cu[num_seqs] != total_tokens) return false;
  for (int64_t r = 0; r < num_seqs; ++r) {
    const int64_t n = host_cu[r + 1] - host_cu[r];
    if (n < 0 || n > max_query_len || host_ctx[r] < 0 || host_ctx[r] + n > max_seq_len) return false;
  }
  return true;
}

// ---------------------------------------------------------------------------
// Host-side argument checks and launchers
// ---------------------------------------------------------------------------
int check_dtype(int dtype) {
  if (dtype != NIE_DTYPE_F32 && dtype != NIE_DTYPE_BF16) {
    return fail(NIE_EUNSUPPORTED, "unsupported dtype code %d", dtype);
  }
  return NIE_OK;
}

int elt_bytes(int dtype) { return dtype == NIE_DTYPE_BF16 ? 2 : 4; }

int check_geometry(int64_t num_layers, int64_t layer_index, int64_t num_blocks,
                   int64_t block_size, int64_t kv_heads, int64_t head_dim) {
  if (num_layers <= 0 || num_blocks <= 0 || block_size <= 0 || kv_heads <= 0 || head_dim <= 0) {
    return fail(NIE_EINVAL, "cache dimensions must be positive");
  }
  if (layer_index < 0 || layer_index >= num_layers) {
    return fail(NIE_EINVAL, "layer_index %lld out of range [0, %lld)", (long long)layer_index,
                (long long)num_layers);
  }
  return NIE_OK;
}

// Shapes the MFMA decode / prefill kernels are built for; every other shape
// of check_attention_shape runs on attention_generic_kernel.
bool tuned_attention(int64_t head_dim, int64_t q_heads, int64_t kv_heads) {
  const int64_t group = q_heads / kv_heads;
  return (head_dim == 64 || head_dim == 128) && (group == 1 || group == 2 || group == 4 || group == 8 || group == 16);
}

int check_attention_shape(int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                          int64_t num_blocks, int64_t block_size) {
  if (head_dim <= 0 || head_dim > kGenericMaxDim) {
    return fail(NIE_EUNSUPPORTED, "head_dim %lld not supported (1 to %d)", (long long)head_dim, kGenericMaxDim);
  }
  if (q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads != 0) {
    return fail(NIE_EINVAL, "q_heads (%lld) must be a positive multiple of kv_heads (%lld)",
                (long long)q_heads, (long long)kv_heads);
  }
  if (num_blocks > 0x7fffffffLL || block_size > 0x7fffffffLL / 16 || kv_heads > 65535) {
    return fail(NIE_EINVAL, "pool dimensions exceed the supported range");
  }
  return NIE_OK;
}

CacheGeom make_geom(int64_t layer_index, int64_t num_blocks, int64_t block_size,
                    int64_t kv_heads, int64_t head_dim) {
  CacheGeom g;
  g.row_elems = kv_heads * head_dim;
  g.layer_offset = layer_index * num_blocks * block_size * g.row_elems;
  g.num_blocks = (int32_t)num_blocks;
  g.block_size = (int32_t)block_size;
  g.bs_shift = -1;
  if ((block_size & (block_size - 1)) == 0) {
    int s = 0;
    while ((1LL << s) < block_size) ++s;
    g.bs_shift = s;
  }
  g.kv_heads = (int32_t)kv_heads;
  g.row_elems32 = (int32_t)g.row_elems;
  return g;
}

// One wave-uniform block lookup per tile needs the tile inside one block:
// block_size a power of two of at least 16.
bool uniform_tiles(const CacheGeom& g) { return g.bs_shift >= 4; }

// Resident decode workgroups per CU of one instantiation: the runtime's
// occupancy figure, or the LDS bound when it cannot be queried.
template <typename T, int D, bool U, int H>
int decode_resident() {
  static const int n = [] {
    int blocks = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, paged_decode_kernel<T, D, U, H>, H * kWave, 0) !=
            hipSuccess ||
        blocks < 1) {
      (void)hipGetLastError();
      constexpr int lds = decode_stages<T, D, H>() * 2 * GroupTile<T, D, H>::kBytes;
      blocks = kDecodeLdsBudget / lds > 0 ? kDecodeLdsBudget / lds : 1;
    }
    return blocks;
  }();
  return n;
}

// Heads per workgroup: the largest power of two that divides kv_heads, up to
// the number that fills a 1 KiB row slice.
template <typename T, int D>
int decode_heads(int64_t kv_heads) {
  constexpr int kMax = decode_max_heads<T, D>();
  const int cap = decode_heads_cap();
  int heads = 1;
  while (heads * 2 <= kMax && heads * 2 <= cap && kv_heads % (heads * 2) == 0) heads *= 2;
  return heads;
}

// Instantiation of a decode launch for a runtime head count.
template <int kMax, int H>
constexpr int heads_clamp() {
  return kMax >= H ? H : 1;
}

template <typename T, int D, bool U>
int decode_resident_u(int heads) {
  constexpr int kMax = decode_max_heads<T, D>();
  switch (heads) {
    case 1: return decode_resident<T, D, U, 1>();
    case 2: return decode_resident<T, D, U, heads_clamp<kMax, 2>()>();
    case 4: return decode_resident<T, D, U, heads_clamp<kMax, 4>()>();
    default: return decode_resident<T, D, U, heads_clamp<kMax, 8>()>();
  }
}

// P: 0 for paged_decode_kernel, else a pass of decode_pass_kernel.
template <typename T, int D, bool U, int H, int P>
void launch_decode_h(const DecodeArgs& a, const DecodeItems& items, int64_t grid_items, hipStream_t stream) {
  const dim3 grid((unsigned)grid_items, (unsigned)(a.geom.kv_heads / H));
  if constexpr (P == 0) {
    if (a.merge_last) {
      hipLaunchKernelGGL((paged_decode_kernel<T, D, U, H, true>), grid, dim3(H * kWave), 0, stream, a, items);
    } else {
      hipLaunchKernelGGL((paged_decode_kernel<T, D, U, H>), grid, dim3(H * kWave), 0, stream, a, items);
    }
  } else {
    hipLaunchKernelGGL((decode_pass_kernel<T, D, U, H, P>), grid, dim3(H * kWave), 0, stream, a, items);
  }
}

template <typename T, int D, bool U, int P = 0>
void launch_decode_u(const DecodeArgs& a, const DecodePlan& p, const DecodeItems& items, hipStream_t stream) {
  constexpr int kMax = decode_max_heads<T, D>();
  const int64_t n = items.count > 0 ? items.count : p.items;
  switch (p.heads) {
    case 1: launch_decode_h<T, D, U, 1, P>(a, items, n, stream); break;
    case 2: launch_decode_h<T, D, U, heads_clamp<kMax, 2>(), P>(a, items, n, stream); break;
    case 4: launch_decode_h<T, D, U, heads_clamp<kMax, 4>(), P>(a, items, n, stream); break;
    default: launch_decode_h<T, D, U, heads_clamp<kMax, 8>(), P>(a, items, n, stream); break;
  }
}

// Without host copies of the lengths the split length is chosen on the
// device, from the lengths themselves (decode_device_tps: the smallest that
// fits one round of `slots` workgroups), so the launch needs no host
// knowledge of them beyond an upper bound on their sum: the grid and the
// workspace cover at most slots - 1 items, or tiles / cap + batch + 1 when
// the split length reaches its cap.  A captured decode step replays with
// the split length its lengths of the moment call for.
template <typename T, int D>
DecodePlan plan_decode_t(int64_t kv_heads, bool uniform, int64_t batch, int64_t total_seq_len) {
  DecodePlan p;
  p.heads = decode_heads<T, D>(kv_heads);
  p.resident = uniform ? decode_resident_u<T, D, true>(p.heads) : decode_resident_u<T, D, false>(p.heads);
  const int64_t groups = kv_heads / p.heads;
  const int64_t cus = device_cus();
  p.slots = (cus * p.resident) / groups > 0 ? (cus * p.resident) / groups : 1;
  p.tps = 0;
  const int64_t capped = decode_max_items(batch, total_seq_len, kDecodeMaxTilesPerSplit);
  p.items = capped > p.slots ? capped : p.slots;
  // at least a full item table: a launch planned from bounds covers (grid
  // and workspace) any host plan a device-resident table may hold
  p.items = p.items > kMaxDecodeItems ? p.items : kMaxDecodeItems;
  const int64_t forced = decode_tiles_override();
  if (forced > 0) {
    p.tps = forced < kDecodeMaxTilesPerSplit ? forced : kDecodeMaxTilesPerSplit;
    p.items = decode_max_items(batch, total_seq_len, p.tps);
  }
  return p;
}

// Work items of host lengths `lens` split into tiles_per_split-tile pieces.
int64_t decode_items_exact(const int32_t* lens, int64_t batch, int64_t tps) {
  int64_t n = 0;
  for (int64_t b = 0; b < batch; ++b) n += cdiv(cdiv((int64_t)lens[b], (int64_t)kTileKeys), tps);
  return n;
}

// The plan from host copies of the lengths: for each number of rounds r the
// smallest split length whose exact item count fits r rounds (the item count
// only falls as the split length grows), then the r with the lowest
// r * (kDecodeFixedTiles + tiles per split), as in plan_decode_t.
DecodePlan plan_decode_exact(DecodePlan p, const int32_t* lens, int64_t batch) {
  const int64_t slots = p.slots;
  p.tps = kDecodeMaxTilesPerSplit;
  int64_t best = -1;
  for (int64_t r = 1; r <= kDecodeMaxRounds; ++r) {
    if (decode_items_exact(lens, batch, kDecodeMaxTilesPerSplit) > r * slots) continue;
    int64_t lo = kDecodeMinTilesPerSplit, hi = kDecodeMaxTilesPerSplit;
    while (lo < hi) {
      const int64_t mid = (lo + hi) / 2;
      if (decode_items_exact(lens, batch, mid) <= r * slots) hi = mid;
      else lo = mid + 1;
    }
    const int64_t cost = r * (kDecodeFixedTiles + lo);
    if (best < 0 || cost < best) {
      best = cost;
      p.tps = lo;
    }
  }
  const int64_t forced = decode_tiles_override();
  if (forced > 0) p.tps = forced < kDecodeMaxTilesPerSplit ? forced : kDecodeMaxTilesPerSplit;
  p.items = decode_items_exact(lens, batch, p.tps);
  return p;
}

// host_lens: optional host copy of the lengths (validated by the caller).
DecodePlan plan_decode(int dtype, int64_t head_dim, int64_t kv_heads, int64_t block_size, int64_t batch,
                       int64_t total_seq_len, const int32_t* host_lens) {
  const bool uniform = block_size >= 16 && (block_size & (block_size - 1)) == 0;
  DecodePlan p;
  if (dtype == NIE_DTYPE_BF16) {
    p = head_dim == 64 ? plan_decode_t<bf16_t, 64>(kv_heads, uniform, batch, total_seq_len)
                       : plan_decode_t<bf16_t, 128>(kv_heads, uniform, batch, total_seq_len);
  } else {
    p = head_dim == 64 ? plan_decode_t<float, 64>(kv_heads, uniform, batch, total_seq_len)
                       : plan_decode_t<float, 128>(kv_heads, uniform, batch, total_seq_len);
  }
  return host_lens != nullptr ? plan_decode_exact(p, host_lens, batch) : p;
}

// The work-item table of a host-planned decode call (count 0 when the call
// does not fit the table: the kernels then locate their work themselves).
void fill_decode_items(const DecodePlan& p, const int32_t* host_lens, int64_t batch, DecodeItems* items) {
  items->count = 0;
  items->tps = (int32_t)p.tps;
  if (host_lens == nullptr || batch > kMaxDecodeSeqs || p.items > kMaxDecodeItems) return;
  int64_t n = 0;
  for (int64_t b = 0; b < batch; ++b) {
    const int64_t nsplit = cdiv(cdiv((int64_t)host_lens[b], (int64_t)kTileKeys), p.tps);
    items->seq_len[b] = host_lens[b];
    items->seq_first[b] = (int32_t)n;
    for (int64_t k = 0; k < nsplit; ++k) items->item[n++] = (uint32_t)((b << 16) | k);
  }
  items->count = (int32_t)n;
}

// Host lengths that match the call: each in [1, max_seq_len], maximum
// max_seq_len, sum total_seq_len.
bool host_lens_ok(const int32_t* lens, int64_t batch, int64_t max_seq_len, int64_t total_seq_len) {
  int64_t sum = 0, mx = 0;
  for (int64_t b = 0; b < batch; ++b) {
    if (lens[b] < 1 || lens[b] > max_seq_len) return false;
    sum += lens[b];
    mx = lens[b] > mx ? lens[b] : mx;
  }
  return sum == total_seq_len && mx == max_seq_len;
}

template <typename T, int D>
void launch_decode(const DecodeArgs& a, const DecodePlan& p, const DecodeItems& items, hipStream_t stream,
                   bool merge) {
  if (uniform_tiles(a.geom)) launch_decode_u<T, D, true>(a, p, items, stream);
  else launch_decode_u<T, D, false>(a, p, items, stream);
  if (merge) {
    const dim3 mgrid((unsigned)a.batch, (unsigned)cdiv((int64_t)a.q_heads, (int64_t)kMergeWaves));
    hipLaunchKernelGGL((decode_merge_kernel<T, D, false>), mgrid, dim3(kMergeWaves * kWave), 0, stream, a, items);
  }
}

// The two-pass rounding: the scores pass (with the fused append and RoPE),
// then the P.V pass over the cache it appended to, then the sum of the
// split partials.
template <typename T, int D>
void launch_decode_two_pass(const DecodeArgs& a, const DecodePlan& p, const DecodeItems& items, hipStream_t stream,
                            bool merge) {
  DecodeArgs pv = a;
  pv.k_new = pv.v_new = nullptr;
  pv.rope_cos = pv.rope_sin = nullptr;
  if (uniform_tiles(a.geom)) {
    launch_decode_u<T, D, true, kDecodeScores>(a, p, items, stream);
    launch_decode_u<T, D, true, kDecodePV>(pv, p, items, stream);
  } else {
    launch_decode_u<T, D, false, kDecodeScores>(a, p, items, stream);
    launch_decode_u<T, D, false, kDecodePV>(pv, p, items, stream);
  }
  if (merge) {
    const dim3 mgrid((unsigned)a.batch, (unsigned)cdiv((int64_t)a.q_heads, (int64_t)kMergeWaves));
    hipLaunchKernelGGL((decode_merge_kernel<T, D, true>), mgrid, dim3(kMergeWaves * kWave), 0, stream, pv, items);
  }
}

// The one-launch decode (decode_fused_kernel), process-wide switch
// (nie_set_decode_fused), and the polls of its waits (nie_set_decode_fused_spin).
std::atomic<int> g_decode_fused{1};
std::atomic<int> g_fused_spin{kFusedSpinLimit};
// Which path the calling thread's last decode call took (nie_decode_last_path).
thread_local int g_decode_path = NIE_DECODE_PATH_NONE;

// Resident decode_fused_kernel workgroups per CU (the runtime's occupancy
// figure, or the LDS bound when it cannot be queried).
template <int H>
int fused_resident() {
  static const int n = [] {
    int blocks = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, decode_fused_kernel<H>, H * kWave, 0) != hipSuccess ||
        blocks < 1) {
      (void)hipGetLastError();
      blocks = kDecodeLdsBudget / (H * kFusedWaveLds) > 0 ? kDecodeLdsBudget / (H * kFusedWaveLds) : 1;
    }
    return blocks;
  }();
  return n;
}

int fused_resident_h(int heads) {
  switch (heads) {
    case 1: return fused_resident<1>();
    case 2: return fused_resident<2>();
    case 4: return fused_resident<4>();
    default: return fused_resident<8>();
  }
}

// Whether decode_fused_kernel runs a reference-rounding call: bf16 head_dim
// 64 on whole-tile blocks, GQA groups of at most kFusedMaxGroup query heads
// (the wave's score region), a counter per (sequence, KV head) in the
// control region, and every work item the launch can hold (`live`, times
// the head groups) resident at once.
bool fused_fits(const CacheGeom& g, const DecodePlan& p, int64_t head_dim, int64_t q_heads, int64_t batch,
                int64_t live) {
  if (g_decode_fused.load(std::memory_order_relaxed) == 0) return false;
  if (head_dim != kFusedDim || !uniform_tiles(g) || q_heads / g.kv_heads > kFusedMaxGroup) return false;
  if (batch * g.kv_heads > kCtlPairs) return false;
  const int64_t groups = g.kv_heads / p.heads;
  return live * groups <= device_cus() * (int64_t)fused_resident_h(p.heads);
}

void launch_decode_fused(const DecodeArgs& a, const DecodePlan& p, const DecodeItems& items, hipStream_t stream) {
  const int64_t n = items.count > 0 ? items.count : p.items;
  const dim3 grid((unsigned)n, (unsigned)(a.geom.kv_heads / p.heads));
  switch (p.heads) {
    case 1: hipLaunchKernelGGL((decode_fused_kernel<1>), grid, dim3(kWave), 0, stream, a, items); break;
    case 2: hipLaunchKernelGGL((decode_fused_kernel<2>), grid, dim3(2 * kWave), 0, stream, a, items); break;
    case 4: hipLaunchKernelGGL((decode_fused_kernel<4>), grid, dim3(4 * kWave), 0, stream, a, items); break;
    default: hipLaunchKernelGGL((decode_fused_kernel<8>), grid, dim3(8 * kWave), 0, stream, a, items); break;
  }
}

template <typename T, int D, int NB, bool P2, int M>
void launch_prefill_kernel(const PrefillArgs& a, const PrefillPlan& p, const PrefillSchedule& sc, hipStream_t stream) {
  const dim3 grid((unsigned)(p.items * a.geom.kv_heads * (M == kPrefillStats ? a.stats_parts : 1)));
  const dim3 block(kPrefillWaves * kWave);
  if (uniform_tiles(a.geom) && p.long_pieces) {
    hipLaunchKernelGGL((varlen_prefill_kernel<T, D, true, NB, P2, M, kPrefillTableWindows>), grid, block, 0, stream,
                       a, sc);
  } else if (uniform_tiles(a.geom)) {
    hipLaunchKernelGGL((varlen_prefill_kernel<T, D, true, NB, P2, M, 1>), grid, block, 0, stream, a, sc);
  } else {
    hipLaunchKernelGGL((varlen_prefill_kernel<T, D, false, NB, P2, M, 1>), grid, block, 0, stream, a, sc);
  }
}

// The reference rounding: the stats pass, then the exact pass.
template <typename T, int D, int NB, bool P2>
void launch_prefill_two_pass(const PrefillArgs& a, const PrefillPlan& p, const PrefillSchedule& sc,
                             hipStream_t stream) {
  launch_prefill_kernel<T, D, NB, P2, kPrefillStats>(a, p, sc, stream);
  launch_prefill_kernel<T, D, NB, P2, kPrefillExact>(a, p, sc, stream);
}

// A positive power of two (the softmax scale of head_dim 64 is 1/8).
bool is_pow2_scale(float scale) {
  int e = 0;
  return scale > 0.f && std::isfinite(scale) && std::frexp(scale, &e) == 0.5f && std::isnormal(scale);
}

template <typename T, int D, int NB, bool kSum>
void launch_prefill_merge(const PrefillArgs& m, const PrefillPlan& p, const PrefillMergeJobs& jobs,
                          hipStream_t stream) {
  const dim3 grid((unsigned)(m.merge_tiles * m.geom.kv_heads * (prefill_rows_per_item<NB>() / kPrefillMergeRows)));
  const dim3 block(kPrefillMergeWaves * kWave);
  // splits per round trip: the call's largest split count, in steps of
  // 4, 8, 16 (8 at head_dim 128); more splits take several round trips
  if (p.max_split <= 4) {
    hipLaunchKernelGGL((prefill_merge_kernel<T, D, NB, 4, kSum>), grid, block, 0, stream, m, jobs);
  } else if constexpr (D > 64) {
    hipLaunchKernelGGL((prefill_merge_kernel<T, D, NB, 8, kSum>), grid, block, 0, stream, m, jobs);
  } else if (p.max_split <= 8) {
    hipLaunchKernelGGL((prefill_merge_kernel<T, D, NB, 8, kSum>), grid, block, 0, stream, m, jobs);
  } else {
    hipLaunchKernelGGL((prefill_merge_kernel<T, D, NB, 16, kSum>), grid, block, 0, stream, m, jobs);
  }
}

template <typename T, int D, int NB>
void launch_prefill_nb(const PrefillArgs& a, const PrefillPlan& p, const PrefillSchedule& sc,
                       const PrefillMergeJobs& jobs, hipStream_t stream, bool merge, bool two) {
  if constexpr (Elt<T>::kIsBf16) {
    if (two) {
      if (is_pow2_scale(a.scale)) launch_prefill_two_pass<T, D, NB, true>(a, p, sc, stream);
      else launch_prefill_two_pass<T, D, NB, false>(a, p, sc, stream);
    } else if (is_pow2_scale(a.scale)) {
      launch_prefill_kernel<T, D, NB, true, kPrefillOnline>(a, p, sc, stream);
    } else {
      launch_prefill_kernel<T, D, NB, false, kPrefillOnline>(a, p, sc, stream);
    }
  } else {
    launch_prefill_kernel<T, D, NB, false, kPrefillOnline>(a, p, sc, stream);
  }
  if (merge) {
    PrefillArgs m = a;
    m.merge_tiles = (int32_t)(jobs.count > 0 ? jobs.count : p.qtiles);
    if (two) launch_prefill_merge<T, D, NB, true>(m, p, jobs, stream);
    else launch_prefill_merge<T, D, NB, false>(m, p, jobs, stream);
  }
}

template <typename T, int D>
void launch_prefill(const PrefillArgs& a, const PrefillPlan& p, const PrefillSchedule& sc,
                    const PrefillMergeJobs& jobs, hipStream_t stream, bool merge, bool two) {
  if (p.row_blocks == 1) launch_prefill_nb<T, D, 1>(a, p, sc, jobs, stream, merge, two);
  else launch_prefill_nb<T, D, 2>(a, p, sc, jobs, stream, merge, two);
}

// Element alignment of the generic path's pointers.
bool elt_aligned(int64_t es, std::initializer_list<const void*> ptrs) {
  for (const void* p : ptrs) {
    if (p != nullptr && ((uintptr_t)p % es) != 0) return false;
  }
  return true;
}

template <typename T>
void launch_generic_attention(const GenericAttnArgs& a, hipStream_t stream) {
  const int64_t waves = a.rows * a.q_heads;
  hipLaunchKernelGGL((attention_generic_kernel<T>), dim3((unsigned)cdiv(waves, (int64_t)kGenericWaves)),
                     dim3(kGenericWaves * kWave), 0, stream, a);
}

int generic_attention(int dtype, const GenericAttnArgs& a, hipStream_t stream) {
  if (a.rows * a.q_heads > 0xffffffffLL) return fail(NIE_EINVAL, "too many query rows");
  if (dtype == NIE_DTYPE_BF16) launch_generic_attention<bf16_t>(a, stream);
  else launch_generic_attention<float>(a, stream);
  return launched("attention_generic");
}

int check_aligned(const void* p, int64_t stride_a, int64_t stride_b, int64_t es) {
  return ((uintptr_t)p % 16) == 0 && ((stride_a * es) % 16) == 0 && ((stride_b * es) % 16) == 0;
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
NIE_API const char* nie_version(void) { return "nie_paged 0.1 gfx950"; }

NIE_API const char* nie_last_error(void) { return g_last_error; }

NIE_API int nie_kv_append(int dtype, const void* k_new, int64_t k_row_stride, const void* v_new,
                          int64_t v_row_stride, const int64_t* slot_mapping, int64_t num_tokens,
                          void* k_cache, void* v_cache, int64_t num_layers, int64_t layer_index,
                          int64_t num_blocks, int64_t block_size, int64_t kv_heads,
                          int64_t head_dim, void* stream) {
  int rc = check_dtype(dtype);
  if (rc) return rc;
  rc = check_geometry(num_layers, layer_index, num_blocks, block_size, kv_heads, head_dim);
  if (rc) return rc;
  if (num_tokens < 0) return fail(NIE_EINVAL, "num_tokens must be non-negative");
  if (num_tokens == 0) return NIE_OK;
  if (!k_new || !v_new || !slot_mapping || !k_cache || !v_cache) {
    return fail(NIE_EINVAL, "null pointer argument");
  }
  if (k_row_stride < kv_heads * head_dim || v_row_stride < kv_heads * head_dim) {
    return fail(NIE_EINVAL, "row strides must cover kv_heads * head_dim elements");
  }
  if (num_tokens > 0x7fffffffLL) return fail(NIE_EINVAL, "too many tokens");
  const int64_t es = elt_bytes(dtype);
  const int64_t row_bytes = kv_heads * head_dim * es;
  const int vec_ok = (row_bytes % 16 == 0) && check_aligned(k_new, k_row_stride, 0, es) &&
                     check_aligned(v_new, v_row_stride, 0, es) &&
                     ((uintptr_t)k_cache % 16 == 0) && ((uintptr_t)v_cache % 16 == 0);
  const int64_t layer_off = layer_index * num_blocks * block_size * row_bytes;
  const int threads = row_bytes / 16 >= 256 ? 256 : 64;
  hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)num_tokens, 2), dim3(threads), 0,
                     (hipStream_t)stream, (const unsigned char*)k_new, k_row_stride * es,
                     (const unsigned char*)v_new, v_row_stride * es, slot_mapping, num_tokens,
                     (unsigned char*)k_cache, (unsigned char*)v_cache, layer_off,
                     num_blocks * block_size, row_bytes, vec_ok);
  return launched("kv_append");
}

NIE_API int nie_kv_gather(int dtype, const void* k_cache, const void* v_cache, int64_t num_layers,
                          int64_t layer_index, int64_t num_blocks, int64_t block_size,
                          int64_t kv_heads, int64_t head_dim, const int32_t* block_table,
                          int64_t num_table_entries, int64_t token_count, void* k_out,
                          void* v_out, void* stream) {
  int rc = check_dtype(dtype);
  if (rc) return rc;
  rc = check_geometry(num_layers, layer_index, num_blocks, block_size, kv_heads, head_dim);
  if (rc) return rc;
  if (token_count < 0) return fail(NIE_EINVAL, "token_count must be non-negative");
  if (token_count == 0) return NIE_OK;
  if (num_table_entries <= 0 || num_table_entries * block_size < token_count) {
    return fail(NIE_EINVAL, "block table does not cover token_count");
  }
  if (!k_cache || !v_cache || !block_table || !k_out || !v_out) {
    return fail(NIE_EINVAL, "null pointer argument");
  }
  if (token_count > 0x7fffffffLL) return fail(NIE_EINVAL, "too many tokens");
  const int64_t es = elt_bytes(dtype);
  const int64_t row_bytes = kv_heads * head_dim * es;
  const int vec_ok = (row_bytes % 16 == 0) && ((uintptr_t)k_out % 16 == 0) &&
                     ((uintptr_t)v_out % 16 == 0) && ((uintptr_t)k_cache % 16 == 0) &&
                     ((uintptr_t)v_cache % 16 == 0);
  const int64_t layer_off = layer_index * num_blocks * block_size * row_bytes;
  hipLaunchKernelGGL(kv_gather_kernel, dim3((unsigned)token_count, 2), dim3(64), 0,
                     (hipStream_t)stream, (const unsigned char*)k_cache,
                     (const unsigned char*)v_cache, layer_off, num_blocks, block_size,
                     block_table, num_table_entries, token_count, (unsigned char*)k_out,
                     (unsigned char*)v_out, row_bytes, vec_ok);
  return launched("kv_gather");
}

NIE_API int nie_kv_copy_blocks(int dtype, const void* src_k, const void* src_v,
                               int64_t src_num_blocks, const int32_t* src_blocks, void* dst_k,
                               void* dst_v, int64_t dst_num_blocks, const int32_t* dst_blocks,
                               int64_t count, int64_t num_layers, int64_t block_size,
                               int64_t kv_heads, int64_t head_dim, void* stream) {
  int rc = check_dtype(dtype);
  if (rc) return rc;
  if (count < 0) return fail(NIE_EINVAL, "count must be non-negative");
  if (count == 0) return NIE_OK;
  if (num_layers <= 0 || block_size <= 0 || kv_heads <= 0 || head_dim <= 0) {
    return fail(NIE_EINVAL, "cache dimensions must be positive");
  }
  if (!src_k || !src_v || !dst_k || !dst_v) return fail(NIE_EINVAL, "null pointer argument");
  if ((src_blocks && src_num_blocks <= 0) || (dst_blocks && dst_num_blocks <= 0)) {
    return fail(NIE_EINVAL, "pool sizes must be positive");
  }
  if (count > 0x7fffffffLL || num_layers > 65535) return fail(NIE_EINVAL, "grid too large");
  const int64_t es = elt_bytes(dtype);
  const int64_t block_bytes = block_size * kv_heads * head_dim * es;
  const int vec_ok = (block_bytes % 16 == 0) && ((uintptr_t)src_k % 16 == 0) &&
                     ((uintptr_t)src_v % 16 == 0) && ((uintptr_t)dst_k % 16 == 0) &&
                     ((uintptr_t)dst_v % 16 == 0);
  hipLaunchKernelGGL(kv_copy_blocks_kernel, dim3((unsigned)count, (unsigned)num_layers, 2),
                     dim3(256), 0, (hipStream_t)stream, (const unsigned char*)src_k,
                     (const unsigned char*)src_v, src_num_blocks, src_blocks,
                     (unsigned char*)dst_k, (unsigned char*)dst_v, dst_num_blocks, dst_blocks,
                     count, block_bytes, vec_ok);
  return launched("kv_copy_blocks");
}

NIE_API int nie_rope_kv_append(int dtype, void* q, int64_t q_stride_t, int64_t q_stride_h, int64_t q_heads,
                               const void* k_new, int64_t k_stride_t, int64_t k_stride_h, const void* v_new,
                               int64_t v_stride_t, int64_t v_stride_h, const int64_t* positions,
                               const int64_t* slot_mapping, int64_t num_tokens, const void* cos_table,
                               const void* sin_table, int64_t table_rows, void* k_cache, void* v_cache,
                               int64_t num_layers, int64_t layer_index, int64_t num_blocks, int64_t block_size,
                               int64_t kv_heads, int64_t head_dim, void* stream) {
  int rc = check_dtype(dtype);
  if (rc) return rc;
  rc = check_geometry(num_layers, layer_index, num_blocks, block_size, kv_heads, head_dim);
  if (rc) return rc;
  if (head_dim % 2 != 0) return fail(NIE_EINVAL, "RoPE needs an even head_dim, got %lld", (long long)head_dim);
  if (num_tokens < 0 || q_heads < 0) return fail(NIE_EINVAL, "num_tokens and q_heads must be non-negative");
  if (num_tokens == 0) return NIE_OK;
  if (!q || !k_new || !v_new || !positions || !slot_mapping || !cos_table || !sin_table || !k_cache || !v_cache) {
    return fail(NIE_EINVAL, "null pointer argument");
  }
  if (table_rows <= 0) return fail(NIE_EINVAL, "the sin/cos table must have at least one row");
  const int64_t heads = q_heads + 2 * kv_heads;
  const int rows_per_block = (head_dim == 64 || head_dim == 128) ? 256 / (int)(head_dim / 2) : 1;
  const int64_t blocks = cdiv(num_tokens * heads, rows_per_block);
  if (heads > 0x7fffffffLL || blocks > 0x7fffffffLL) return fail(NIE_EINVAL, "too many tokens");
  RopeAppendArgs a;
  a.q = q;
  a.q_st = q_stride_t;
  a.q_sh = q_stride_h;
  a.k = k_new;
  a.k_st = k_stride_t;
  a.k_sh = k_stride_h;
  a.v = v_new;
  a.v_st = v_stride_t;
  a.v_sh = v_stride_h;
  a.positions = positions;
  a.slots = slot_mapping;
  a.num_tokens = num_tokens;
  a.cos_table = cos_table;
  a.sin_table = sin_table;
  a.table_rows = table_rows;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.layer_offset = layer_index * num_blocks * block_size * kv_heads * head_dim;
  a.pool_slots = num_blocks * block_size;
  a.q_heads = (int32_t)q_heads;
  a.kv_heads = (int32_t)kv_heads;
  hipStream_t s = (hipStream_t)stream;
  if (head_dim != 64 && head_dim != 128) {
    // other even head_dims: one thread per (token, head, pair)
    const int64_t threads = num_tokens * heads * (head_dim / 2);
    if (cdiv(threads, (int64_t)256) > 0x7fffffffLL) return fail(NIE_EINVAL, "too many tokens");
    const dim3 ggrid((unsigned)cdiv(threads, (int64_t)256));
    if (dtype == NIE_DTYPE_BF16) hipLaunchKernelGGL((rope_kv_append_generic_kernel<bf16_t>), ggrid, dim3(256), 0, s, a, (int)head_dim);
    else hipLaunchKernelGGL((rope_kv_append_generic_kernel<float>), ggrid, dim3(256), 0, s, a, (int)head_dim);
    return launched("rope_kv_append");
  }
  const dim3 grid((unsigned)blocks);
  if (dtype == NIE_DTYPE_BF16) {
    if (head_dim == 64) hipLaunchKernelGGL((rope_kv_append_kernel<bf16_t, 64>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((rope_kv_append_kernel<bf16_t, 128>), grid, dim3(256), 0, s, a);
  } else {
    if (head_dim == 64) hipLaunchKernelGGL((rope_kv_append_kernel<float, 64>), grid, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((rope_kv_append_kernel<float, 128>), grid, dim3(256), 0, s, a);
  }
  return launched("rope_kv_append");
}

NIE_API int nie_argmax_rows(int dtype, const void* logits, int64_t rows, int64_t cols, int64_t row_stride,
                            int64_t* out, void* stream) {
  int rc = check_dtype(dtype);
  if (rc) return rc;
  if (rows < 0 || cols <= 0 || row_stride < cols) return fail(NIE_EINVAL, "bad logits shape");
  if (rows == 0) return NIE_OK;
  if (!logits || !out) return fail(NIE_EINVAL, "null pointer argument");
  if (rows > 0x7fffffffLL) return fail(NIE_EINVAL, "too many rows");
  if (dtype == NIE_DTYPE_BF16) {
    hipLaunchKernelGGL(argmax_rows_kernel<bf16_t>, dim3((unsigned)rows), dim3(kArgmaxThreads), 0,
                       (hipStream_t)stream, logits, row_stride, cols, out, nullptr);
  } else {
    hipLaunchKernelGGL(argmax_rows_kernel<float>, dim3((unsigned)rows), dim3(kArgmaxThreads), 0,
                       (hipStream_t)stream, logits, row_stride, cols, out, nullptr);
  }
  return launched("argmax_rows");
}

NIE_API int64_t nie_argmax_rows_workspace_bytes(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  return rows * cdiv(cols, kArgmaxPieceCols) * (int64_t)sizeof(ArgmaxPartial);
}

NIE_API int nie_argmax_rows_split(int dtype, const void* logits, int64_t rows, int64_t cols, int64_t row_stride,
                                  int64_t* out, void* workspace, int64_t workspace_bytes, void* stream) {
  int rc = check_dtype(dtype);
  if (rc) return rc;
  if (rows < 0 || cols <= 0 || row_stride < cols) return fail(NIE_EINVAL, "bad logits shape");
  if (rows == 0) return NIE_OK;
  if (!logits || !out || !workspace) return fail(NIE_EINVAL, "null pointer argument");
  const int64_t pieces = cdiv(cols, kArgmaxPieceCols);
  if (rows > 0x7fffffffLL || pieces > 0xffffLL) return fail(NIE_EINVAL, "too many rows or columns");
  if (workspace_bytes < nie_argmax_rows_workspace_bytes(rows, cols) || ((uintptr_t)workspace % 16) != 0) {
    return fail(NIE_EINVAL, "argmax_rows_split: workspace too small or misaligned");
  }
  ArgmaxPartial* part = reinterpret_cast<ArgmaxPartial*>(workspace);
  const dim3 grid((unsigned)rows, (unsigned)pieces);
  if (dtype == NIE_DTYPE_BF16) {
    hipLaunchKernelGGL(argmax_rows_kernel<bf16_t>, grid, dim3(kArgmaxThreads), 0, (hipStream_t)stream, logits,
                       row_stride, cols, out, part);
  } else {
    hipLaunchKernelGGL(argmax_rows_kernel<float>, grid, dim3(kArgmaxThreads), 0, (hipStream_t)stream, logits,
                       row_stride, cols, out, part);
  }
  rc = launched("argmax_rows");
  if (rc) return rc;
  hipLaunchKernelGGL(argmax_merge_kernel, dim3((unsigned)rows), dim3(kWave), 0, (hipStream_t)stream, part, pieces,
                     out);
  return launched("argmax_merge");
}

NIE_API int nie_rms_norm(int dtype, const void* x, int64_t x_stride, const void* residual,
                         int64_t residual_stride, void* sum_out, int64_t sum_stride, const void* weight,
                         void* out, int64_t out_stride, int64_t rows, int64_t cols, float eps, void* stream) {
  int rc = check_dtype(dtype);
  if (rc) return rc;
  const int64_t es = elt_bytes(dtype);
  const int64_t per_vec = 16 / es;
  if (rows < 0 || cols <= 0 || cols % per_vec != 0 || cols > kNormThreads * kNormVecsPerThread * per_vec) {
    return fail(NIE_EUNSUPPORTED, "rms_norm: %lld columns (need a multiple of %lld, at most %lld)", (long long)cols,
                (long long)per_vec, (long long)(kNormThreads * kNormVecsPerThread * per_vec));
  }
  if (rows == 0) return NIE_OK;
  if (!x || !out || (residual != nullptr && !sum_out)) return fail(NIE_EINVAL, "null pointer argument");
  if (!check_aligned(x, x_stride, 0, es) || !check_aligned(out, out_stride, 0, es) ||
      (residual && (!check_aligned(residual, residual_stride, 0, es) || !check_aligned(sum_out, sum_stride, 0, es))) ||
      (weight && ((uintptr_t)weight % 16))) {
    return fail(NIE_EINVAL, "rms_norm: rows and weight must be 16-byte aligned");
  }
  if (x_stride < cols || out_stride < cols || (residual && (residual_stride < cols || sum_stride < cols))) {
    return fail(NIE_EINVAL, "rms_norm: row strides shorter than the rows");
  }
  if (rows > 0x7fffffffLL) return fail(NIE_EINVAL, "too many rows");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == NIE_DTYPE_BF16) {
    hipLaunchKernelGGL(rms_norm_kernel<bf16_t>, dim3((unsigned)rows), dim3(kNormThreads), 0, s, x, x_stride, residual,
                       residual_stride, sum_out, sum_stride, weight, out, out_stride, (int)cols, eps);
  } else {
    hipLaunchKernelGGL(rms_norm_kernel<float>, dim3((unsigned)rows), dim3(kNormThreads), 0, s, x, x_stride, residual,
                       residual_stride, sum_out, sum_stride, weight, out, out_stride, (int)cols, eps);
  }
  return launched("rms_norm");
}

namespace {

int check_linear(int dtype, const void* x, int64_t x_stride, int64_t rows, const void* w, int64_t n, int64_t k,
                 int epilogue, void* y, int64_t y_stride) {
  int rc = check_dtype(dtype);
  if (rc) return rc;
  if (dtype != NIE_DTYPE_BF16) return fail(NIE_EUNSUPPORTED, "linear_rows: only bf16 is built");
  if (epilogue != NIE_LINEAR_PLAIN && epilogue != NIE_LINEAR_SILU_MUL) {
    return fail(NIE_EINVAL, "linear_rows: unknown epilogue %d", epilogue);
  }
  if (rows < 1 || rows > kLinearMaxRows) {
    return fail(NIE_EUNSUPPORTED, "linear_rows: %lld rows (1..%d are built)", (long long)rows, kLinearMaxRows);
  }
  if (n <= 0 || n % 16 != 0 || n / 16 > 0x7fffffffLL) {
    return fail(NIE_EUNSUPPORTED, "linear_rows: %lld output columns (need a positive multiple of 16)", (long long)n);
  }
  if (k != 2048 && k != 4096 && (k != 8192 || epilogue == NIE_LINEAR_SILU_MUL)) {
    return fail(NIE_EUNSUPPORTED, "linear_rows: inner size %lld (2048, 4096 and, without the SiLU epilogue, 8192 are built)",
                (long long)k);
  }
  if (!x || !w || !y) return fail(NIE_EINVAL, "null pointer argument");
  if (x_stride < k || y_stride < n) return fail(NIE_EINVAL, "linear_rows: row strides shorter than the rows");
  if (!check_aligned(x, x_stride, 0, 2) || !check_aligned(w, 0, 0, 2) || ((uintptr_t)y % 2) != 0) {
    return fail(NIE_EINVAL, "linear_rows: x rows and the weight must be 16-byte aligned");
  }
  return NIE_OK;
}

LinearArgs linear_args(const void* x, int64_t x_stride, int64_t rows, const void* w, int64_t n, int64_t k, void* y,
                       int64_t y_stride) {
  LinearArgs a;
  a.x = reinterpret_cast<const bf16_t*>(x);
  a.x_stride = x_stride;
  a.rows = (int32_t)rows;
  a.w = reinterpret_cast<const bf16_t*>(w);
  a.n = n;
  a.k = k;
  a.y = reinterpret_cast<bf16_t*>(y);
  a.y_stride = y_stride;
  a.res = nullptr;
  a.res_stride = 0;
  a.sum_out = nullptr;
  a.sum_stride = 0;
  a.norm_w = nullptr;
  a.eps = 0.f;
  return a;
}

template <bool kNorm>
int launch_linear(const LinearArgs& a, int epilogue, hipStream_t s) {
  // one workgroup per CU (the ring takes 128 KiB of LDS), at most one per tile
  const int64_t tiles = a.n / 16;
  const int64_t cus = device_cus();
  const dim3 grid((unsigned)(tiles < cus ? tiles : cus)), block(kLinearWaves * kWave);
  const bool silu = epilogue == NIE_LINEAR_SILU_MUL;
  if constexpr (kNorm) {
    if (a.res != nullptr) {
      if (silu) hipLaunchKernelGGL((linear_rows_kernel<kLinearSiluMul, 2, kLinearNormRes>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((linear_rows_kernel<kLinearPlain, 2, kLinearNormRes>), grid, block, 0, s, a);
    } else {
      if (silu) hipLaunchKernelGGL((linear_rows_kernel<kLinearSiluMul, 2, kLinearNorm>), grid, block, 0, s, a);
      else hipLaunchKernelGGL((linear_rows_kernel<kLinearPlain, 2, kLinearNorm>), grid, block, 0, s, a);
    }
  } else {
    switch (a.k) {
      case 2048:
        if (silu) hipLaunchKernelGGL((linear_rows_kernel<kLinearSiluMul, 2, kLinearNoNorm>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((linear_rows_kernel<kLinearPlain, 2, kLinearNoNorm>), grid, block, 0, s, a);
        break;
      case 4096:
        if (silu) hipLaunchKernelGGL((linear_rows_kernel<kLinearSiluMul, 4, kLinearNoNorm>), grid, block, 0, s, a);
        else hipLaunchKernelGGL((linear_rows_kernel<kLinearPlain, 4, kLinearNoNorm>), grid, block, 0, s, a);
        break;
      default:
        hipLaunchKernelGGL((linear_rows_kernel<kLinearPlain, 8, kLinearNoNorm>), grid, block, 0, s, a);
        break;
    }
  }
  return launched("linear_rows_kernel");
}

}  // namespace

NIE_API int nie_linear_rows(int dtype, const void* x, int64_t x_stride, int64_t rows, const void* w, int64_t n,
                            int64_t k, int epilogue, void* y, int64_t y_stride, void* stream) {
  const int rc = check_linear(dtype, x, x_stride, rows, w, n, k, epilogue, y, y_stride);
  if (rc) return rc;
  return launch_linear<false>(linear_args(x, x_stride, rows, w, n, k, y, y_stride), epilogue, (hipStream_t)stream);
}

NIE_API int nie_rms_norm_linear_rows(int dtype, const void* x, int64_t x_stride, const void* residual,
                                     int64_t residual_stride, void* sum_out, int64_t sum_stride,
                                     const void* norm_weight, float eps, int64_t rows, const void* w, int64_t n,
                                     int64_t k, int epilogue, void* y, int64_t y_stride, void* stream) {
  const int rc = check_linear(dtype, x, x_stride, rows, w, n, k, epilogue, y, y_stride);
  if (rc) return rc;
  if (k != 2048) return fail(NIE_EUNSUPPORTED, "rms_norm_linear_rows: inner size %lld (2048 is built)", (long long)k);
  if (!norm_weight) return fail(NIE_EINVAL, "rms_norm_linear_rows: null norm weight");
  if (!(eps >= 0.f) || !std::isfinite(eps)) return fail(NIE_EINVAL, "rms_norm_linear_rows: eps must be finite and >= 0");
  if (!check_aligned(norm_weight, 0, 0, 2)) return fail(NIE_EINVAL, "rms_norm_linear_rows: misaligned norm weight");
  if (residual != nullptr && (residual_stride < k || !check_aligned(residual, residual_stride, 0, 2))) {
    return fail(NIE_EINVAL, "rms_norm_linear_rows: residual rows shorter than k or misaligned");
  }
  if (sum_out != nullptr && (residual == nullptr || sum_stride < k || !check_aligned(sum_out, sum_stride, 0, 2))) {
    return fail(NIE_EINVAL, "rms_norm_linear_rows: sum_out needs a residual and aligned rows of k elements");
  }
  LinearArgs a = linear_args(x, x_stride, rows, w, n, k, y, y_stride);
  a.res = reinterpret_cast<const bf16_t*>(residual);
  a.res_stride = residual_stride;
  a.sum_out = reinterpret_cast<bf16_t*>(sum_out);
  a.sum_stride = sum_stride;
  a.norm_w = reinterpret_cast<const bf16_t*>(norm_weight);
  a.eps = eps;
  return launch_linear<true>(a, epilogue, (hipStream_t)stream);
}

NIE_API int nie_silu_mul(int dtype, const void* gate, int64_t gate_stride, const void* up, int64_t up_stride,
                         void* out, int64_t out_stride, int64_t rows, int64_t cols, void* stream) {
  int rc = check_dtype(dtype);
  if (rc) return rc;
  const int64_t es = elt_bytes(dtype);
  const int64_t per_vec = 16 / es;
  if (rows < 0 || cols <= 0 || cols % per_vec != 0) {
    return fail(NIE_EUNSUPPORTED, "silu_mul: rows of %lld elements (need a multiple of %lld)", (long long)cols,
                (long long)per_vec);
  }
  if (rows == 0) return NIE_OK;
  if (!gate || !up || !out) return fail(NIE_EINVAL, "null pointer argument");
  if (!check_aligned(gate, gate_stride, 0, es) || !check_aligned(up, up_stride, 0, es) ||
      !check_aligned(out, out_stride, 0, es)) {
    return fail(NIE_EINVAL, "silu_mul: rows must be 16-byte aligned");
  }
  if ((rows > 1 && (gate_stride < cols || up_stride < cols || out_stride < cols))) {
    return fail(NIE_EINVAL, "silu_mul: row strides shorter than the rows");
  }
  const int64_t vecs_per_row = cols / per_vec;
  const int64_t nvec = rows * vecs_per_row;
  const int64_t blocks = cdiv(nvec, (int64_t)256);
  if (blocks > 0x7fffffffLL) return fail(NIE_EINVAL, "silu_mul: too many elements");
  hipStream_t s = (hipStream_t)stream;
  if (dtype == NIE_DTYPE_BF16) {
    hipLaunchKernelGGL(silu_mul_kernel<bf16_t>, dim3((unsigned)blocks), dim3(256), 0, s, gate, gate_stride, up,
                       up_stride, out, out_stride, vecs_per_row, nvec);
  } else {
    hipLaunchKernelGGL(silu_mul_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, s, gate, gate_stride, up,
                       up_stride, out, out_stride, vecs_per_row, nvec);
  }
  return launched("silu_mul");
}

NIE_API int64_t nie_paged_decode_workspace_bytes(int dtype, int64_t batch, int64_t q_heads,
                                                 int64_t kv_heads, int64_t head_dim,
                                                 int64_t block_size, int64_t max_seq_len,
                                                 int64_t total_seq_len, const int32_t* host_seq_lens) {
  if (check_dtype(dtype) != NIE_OK || batch <= 0 || q_heads <= 0 || total_seq_len <= 0 || block_size <= 0 ||
      check_attention_shape(q_heads, kv_heads, head_dim, 1, block_size) != NIE_OK) {
    return 0;
  }
  if (host_seq_lens != nullptr && !host_lens_ok(host_seq_lens, batch, max_seq_len, total_seq_len)) return 0;
  if (!tuned_attention(head_dim, q_heads, kv_heads)) return 0;  // the generic kernel needs no workspace
  const DecodePlan p = plan_decode(dtype, head_dim, kv_heads, block_size, batch, total_seq_len, host_seq_lens);
  return kCtlBytes + decode_workspace_need(p, q_heads, head_dim, batch, total_seq_len, two_pass(dtype));
}

NIE_API int nie_set_attention_rounding(int mode) {
  if (mode != NIE_ROUND_REFERENCE && mode != NIE_ROUND_FAST) {
    return fail(NIE_EINVAL, "attention rounding must be NIE_ROUND_REFERENCE or NIE_ROUND_FAST");
  }
  g_rounding.store(mode, std::memory_order_relaxed);
  return NIE_OK;
}

NIE_API int nie_attention_rounding(void) { return g_rounding.load(std::memory_order_relaxed); }

NIE_API int nie_set_decode_fused(int on) {
  if (on < 0 || on > 2) return fail(NIE_EINVAL, "nie_set_decode_fused takes 0, 1 or 2");
  g_decode_fused.store(on, std::memory_order_relaxed);
  return NIE_OK;
}

NIE_API int nie_decode_fused(void) { return g_decode_fused.load(std::memory_order_relaxed); }

NIE_API int nie_set_decode_fused_spin(int polls) {
  if (polls < 0) return fail(NIE_EINVAL, "nie_set_decode_fused_spin takes a non-negative poll count");
  g_fused_spin.store(polls, std::memory_order_relaxed);
  return NIE_OK;
}

NIE_API int64_t nie_workspace_control_bytes(void) { return kCtlBytes; }

NIE_API int nie_decode_last_path(void) { return g_decode_path; }

namespace {

// New K/V rows of a fused decode step (nie_paged_decode_append).
struct DecodeAppend {
  const void* k_new = nullptr;
  int64_t k_stride = 0;
  const void* v_new = nullptr;
  int64_t v_stride = 0;
  const void* cos_table = nullptr;  // RoPE tables (table_rows, head_dim / 2); nullptr: no RoPE
  const void* sin_table = nullptr;
  int64_t table_rows = 0;
};

int paged_decode_call(int dtype, const void* q, int64_t q_stride_b, int64_t q_stride_h, const void* k_cache,
                      const void* v_cache, int64_t num_layers, int64_t layer_index, int64_t num_blocks,
                      int64_t block_size, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                      const int32_t* block_tables, int64_t table_stride, const int32_t* seq_lens, int64_t batch,
                      int64_t max_seq_len, int64_t total_seq_len, float scale, void* out, int64_t out_stride_b,
                      int64_t out_stride_h, void* workspace, int64_t workspace_bytes,
                      const int32_t* host_seq_lens, const DecodeAppend& append, void* stream,
                      bool static_scratch = false, const void* device_plan = nullptr) {
  g_decode_path = NIE_DECODE_PATH_NONE;
  int rc = check_dtype(dtype);
  if (rc) return rc;
  rc = check_geometry(num_layers, layer_index, num_blocks, block_size, kv_heads, head_dim);
  if (rc) return rc;
  rc = check_attention_shape(q_heads, kv_heads, head_dim, num_blocks, block_size);
  if (rc) return rc;
  if (batch < 0) return fail(NIE_EINVAL, "batch must be non-negative");
  if (batch == 0) return NIE_OK;
  if (!q || !k_cache || !v_cache || !block_tables || !seq_lens || !out) {
    return fail(NIE_EINVAL, "null pointer argument");
  }
  if (max_seq_len <= 0 || max_seq_len > 0x7fffffffLL - kTileKeys || total_seq_len < max_seq_len ||
      total_seq_len > max_seq_len * batch) {
    return fail(NIE_EINVAL, "inconsistent max_seq_len / total_seq_len");
  }
  if (table_stride <= 0 || table_stride > 0x7fffffffLL || table_stride * block_size < max_seq_len) {
    return fail(NIE_EINVAL, "block table row (%lld entries) does not cover max_seq_len (%lld)",
                (long long)table_stride, (long long)max_seq_len);
  }
  const int64_t es = elt_bytes(dtype);
  if (!tuned_attention(head_dim, q_heads, kv_heads)) {
    // other shapes: the generic kernels (no workspace; element alignment)
    if (!elt_aligned(es, {q, out, k_cache, v_cache, append.k_new, append.v_new, append.cos_table, append.sin_table})) {
      return fail(NIE_EINVAL, "pointers must be aligned to the element size");
    }
    if (append.k_new != nullptr || append.v_new != nullptr) {
      if (!append.k_new || !append.v_new) return fail(NIE_EINVAL, "null pointer argument");
      if (append.k_stride < kv_heads * head_dim || append.v_stride < kv_heads * head_dim) {
        return fail(NIE_EINVAL, "new K/V rows must be (batch, kv_heads, head_dim) rows");
      }
      if (append.cos_table != nullptr || append.sin_table != nullptr) {
        if (!append.cos_table || !append.sin_table || append.table_rows <= 0) {
          return fail(NIE_EINVAL, "RoPE needs both tables and at least one row");
        }
        if (head_dim % 2) return fail(NIE_EINVAL, "RoPE needs an even head_dim");
      }
    }
    if (batch > 0x7fffffffLL) return fail(NIE_EINVAL, "batch too large");
    const CacheGeom geom = make_geom(layer_index, num_blocks, block_size, kv_heads, head_dim);
    hipStream_t s = (hipStream_t)stream;
    if (append.k_new != nullptr) {
      GenericAppendArgs g;
      g.k_new = append.k_new;
      g.kn_s = append.k_stride;
      g.v_new = append.v_new;
      g.vn_s = append.v_stride;
      g.k_cache = const_cast<void*>(k_cache);
      g.v_cache = const_cast<void*>(v_cache);
      g.geom = geom;
      g.head_dim = (int32_t)head_dim;
      g.tables = block_tables;
      g.table_stride = table_stride;
      g.seq_lens = seq_lens;
      g.batch = batch;
      g.rope_cos = append.cos_table;
      g.rope_sin = append.sin_table;
      g.rope_rows = append.table_rows;
      const dim3 grid((unsigned)cdiv(batch * kv_heads * head_dim, (int64_t)256));
      if (dtype == NIE_DTYPE_BF16) hipLaunchKernelGGL((decode_append_generic_kernel<bf16_t>), grid, dim3(256), 0, s, g);
      else hipLaunchKernelGGL((decode_append_generic_kernel<float>), grid, dim3(256), 0, s, g);
      rc = launched("decode_append_generic");
      if (rc) return rc;
    }
    GenericAttnArgs ga{};
    ga.q = q;
    ga.q_sr = q_stride_b;
    ga.q_sh = q_stride_h;
    ga.out = out;
    ga.o_sr = out_stride_b;
    ga.o_sh = out_stride_h;
    ga.k_cache = k_cache;
    ga.v_cache = v_cache;
    ga.geom = geom;
    ga.head_dim = (int32_t)head_dim;
    ga.q_heads = (int32_t)q_heads;
    ga.group = (int32_t)(q_heads / kv_heads);
    ga.tables = block_tables;
    ga.table_stride = table_stride;
    ga.scale = scale;
    ga.rows = batch;
    ga.seq_lens = seq_lens;
    ga.rope_cos = append.k_new != nullptr ? append.cos_table : nullptr;
    ga.rope_sin = append.k_new != nullptr ? append.sin_table : nullptr;
    ga.rope_rows = append.table_rows;
    g_decode_path = NIE_DECODE_PATH_GENERIC;
    return generic_attention(dtype, ga, s);
  }
  if (!check_aligned(q, q_stride_b, q_stride_h, es) || !check_aligned(out, out_stride_b, out_stride_h, es) ||
      ((uintptr_t)k_cache % 16) || ((uintptr_t)v_cache % 16)) {
    return fail(NIE_EINVAL, "q/out/cache pointers and strides must be 16-byte aligned");
  }
  if (host_seq_lens != nullptr && !host_lens_ok(host_seq_lens, batch, max_seq_len, total_seq_len)) {
    return fail(NIE_EINVAL, "host seq_lens do not match max_seq_len / total_seq_len");
  }
  if (append.k_new != nullptr || append.v_new != nullptr) {
    if (!append.k_new || !append.v_new) return fail(NIE_EINVAL, "null pointer argument");
    if (append.k_stride < kv_heads * head_dim || append.v_stride < kv_heads * head_dim ||
        !check_aligned(append.k_new, append.k_stride, head_dim, es) ||
        !check_aligned(append.v_new, append.v_stride, head_dim, es)) {
      return fail(NIE_EINVAL, "new K/V rows must be 16-byte aligned (batch, kv_heads, head_dim) rows");
    }
    if (append.cos_table != nullptr || append.sin_table != nullptr) {
      if (!append.cos_table || !append.sin_table || append.table_rows <= 0) {
        return fail(NIE_EINVAL, "RoPE needs both tables and at least one row");
      }
      if (((uintptr_t)append.cos_table % 16) || ((uintptr_t)append.sin_table % 16)) {
        return fail(NIE_EINVAL, "RoPE tables must be 16-byte aligned");
      }
    }
  }
  const DecodePlan plan = plan_decode(dtype, head_dim, kv_heads, block_size, batch, total_seq_len, host_seq_lens);
  const int64_t tps = plan.tps;  // 0: chosen on the device, at least kDecodeMinTilesPerSplit
  const int64_t items = plan.items;
  const bool may_split = cdiv(max_seq_len, kTileKeys) > (tps > 0 ? tps : kDecodeMinTilesPerSplit);
  // the two-pass rounding always needs the workspace (its score buffer and
  // the (max, sum) pairs of every split, one split included)
  const bool two = two_pass(dtype);
  // the workspace: the control region, then the partials (and scores)
  const int64_t need = kCtlBytes + decode_workspace_need(plan, q_heads, head_dim, batch, total_seq_len, two);
  if ((may_split || two) && (workspace == nullptr || workspace_bytes < need || ((uintptr_t)workspace % 16))) {
    if (static_scratch) {
      return fail(NIE_EINVAL,
                  "split partials need %lld bytes, beyond the %lld-byte static scratch of the allocation-free "
                  "entry point; call nie_paged_decode_append with a workspace instead",
                  (long long)need, (long long)workspace_bytes);
    }
    return fail(NIE_EINVAL, "workspace too small: need %lld bytes, got %lld", (long long)need,
                (long long)workspace_bytes);
  }
  if (items > 0x7fffffffLL || batch > 0x7fffffffLL) return fail(NIE_EINVAL, "batch too large");
  DecodeArgs a;
  a.q = q;
  a.q_sb = q_stride_b;
  a.q_sh = q_stride_h;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.geom = make_geom(layer_index, num_blocks, block_size, kv_heads, head_dim);
  a.q_heads = (int32_t)q_heads;
  a.group = (int32_t)(q_heads / kv_heads);
  a.tables = block_tables;
  a.table_stride = table_stride;
  a.seq_lens = seq_lens;
  a.batch = batch;
  a.tiles_per_split = (int32_t)tps;
  a.split_slots = (int32_t)plan.slots;
  a.dev_items = reinterpret_cast<const DecodeItems*>(device_plan);
  a.scale = scale;
  a.out = out;
  a.o_sb = out_stride_b;
  a.o_sh = out_stride_h;
  const bool have_ws = workspace != nullptr && workspace_bytes >= need;
  unsigned char* const body = have_ws ? reinterpret_cast<unsigned char*>(workspace) + kCtlBytes : nullptr;
  a.ctl = have_ws ? reinterpret_cast<DecodeCtl*>(workspace) : nullptr;
  a.spin_limit = g_fused_spin.load(std::memory_order_relaxed);
  a.ws_o = have_ws ? reinterpret_cast<float*>(body) : nullptr;
  a.ws_ml = have_ws ? a.ws_o + items * q_heads * head_dim : nullptr;
  a.ws_items = have_ws ? items : 0;
  if (two && have_ws) {
    a.ws_s = reinterpret_cast<uint16_t*>(body + decode_ws_partials(plan, q_heads, head_dim));
    a.ws_s_keys = decode_score_keys(plan, batch, total_seq_len);
  }
  a.k_new = append.k_new;
  a.v_new = append.v_new;
  a.kn_s = append.k_stride;
  a.vn_s = append.v_stride;
  a.rope_cos = append.cos_table;
  a.rope_sin = append.sin_table;
  a.rope_rows = append.table_rows;
  // The grid is an upper bound on the item count (exact to within `batch`);
  // workgroups past the last real item return immediately.
  DecodeItems work;
  fill_decode_items(plan, host_seq_lens, batch, &work);
  hipStream_t s = (hipStream_t)stream;
  if (two) {
    // the most work items the launch can hold: the host plan's, or (the
    // split length chosen on the device) what decode_device_tps allows,
    // and with a device-resident plan whatever that table may hold
    int64_t live = work.count > 0 ? work.count
                   : plan.tps > 0 ? plan.items
                                  : std::max(plan.slots - 1,
                                             decode_max_items(batch, total_seq_len, kDecodeMaxTilesPerSplit));
    if (device_plan != nullptr) live = std::max(live, (int64_t)kMaxDecodeItems);
    if (have_ws && fused_fits(a.geom, plan, head_dim, q_heads, batch, live)) {
      g_decode_path = NIE_DECODE_PATH_FUSED;
      launch_decode_fused(a, plan, work, s);
    } else {
      g_decode_path = NIE_DECODE_PATH_PASSES;
      if (head_dim == 64) launch_decode_two_pass<bf16_t, 64>(a, plan, work, s, may_split);
      else launch_decode_two_pass<bf16_t, 128>(a, plan, work, s, may_split);
    }
  } else {
    // The split that finishes last merges its sequence's partials (a counter
    // per (sequence, KV head) in the control region), or a merge launch does.
    // The merge at the end of a split costs three dependent memory round
    // trips (the partial's write-through, the count, the other partials):
    // cheaper than a merge launch only while the memory system is quiet,
    // i.e. for calls of at most a quarter of the CUs' workgroups (the
    // 4-sequence decode: 16.5 -> 14.5 us per call; the 16-sequence step
    // and 16 x 29600 were 3 us slower with it).
    // (Switch value 2 merges by the last split in calls of every size.)
    const int fused = g_decode_fused.load(std::memory_order_relaxed);
    const int64_t wgs = (work.count > 0 ? work.count : items) * (kv_heads / plan.heads);
    a.merge_last = may_split && have_ws && fused != 0 && batch * kv_heads <= kCtlPairs &&
                   (fused == 2 || wgs <= device_cus() / 4);
    const bool merge = may_split && !a.merge_last;
    g_decode_path = a.merge_last ? NIE_DECODE_PATH_ONE_PASS_MERGED : NIE_DECODE_PATH_ONE_PASS;
    if (dtype == NIE_DTYPE_BF16) {
      if (head_dim == 64) launch_decode<bf16_t, 64>(a, plan, work, s, merge);
      else launch_decode<bf16_t, 128>(a, plan, work, s, merge);
    } else {
      if (head_dim == 64) launch_decode<float, 64>(a, plan, work, s, merge);
      else launch_decode<float, 128>(a, plan, work, s, merge);
    }
  }
  return launched("paged_decode");
}

}  // namespace

NIE_API int nie_paged_decode(int dtype, const void* q, int64_t q_stride_b, int64_t q_stride_h,
                             const void* k_cache, const void* v_cache, int64_t num_layers,
                             int64_t layer_index, int64_t num_blocks, int64_t block_size,
                             int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                             const int32_t* block_tables, int64_t table_stride,
                             const int32_t* seq_lens, int64_t batch, int64_t max_seq_len,
                             int64_t total_seq_len, float scale, void* out,
                             int64_t out_stride_b, int64_t out_stride_h, void* workspace,
                             int64_t workspace_bytes, const int32_t* host_seq_lens, void* stream) {
  return paged_decode_call(dtype, q, q_stride_b, q_stride_h, k_cache, v_cache, num_layers, layer_index, num_blocks,
                           block_size, q_heads, kv_heads, head_dim, block_tables, table_stride, seq_lens, batch,
                           max_seq_len, total_seq_len, scale, out, out_stride_b, out_stride_h, workspace,
                           workspace_bytes, host_seq_lens, DecodeAppend{}, stream);
}

NIE_API int nie_paged_decode_append(int dtype, const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                    const void* k_new, int64_t k_new_stride, const void* v_new,
                                    int64_t v_new_stride, const void* cos_table, const void* sin_table,
                                    int64_t table_rows, void* k_cache, void* v_cache, int64_t num_layers,
                                    int64_t layer_index, int64_t num_blocks, int64_t block_size,
                                    int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                    const int32_t* block_tables, int64_t table_stride,
                                    const int32_t* seq_lens, int64_t batch, int64_t max_seq_len,
                                    int64_t total_seq_len, float scale, void* out, int64_t out_stride_b,
                                    int64_t out_stride_h, void* workspace, int64_t workspace_bytes,
                                    const int32_t* host_seq_lens, void* stream) {
  if (batch > 0 && (!k_new || !v_new)) return fail(NIE_EINVAL, "null pointer argument");
  DecodeAppend append;
  append.k_new = k_new;
  append.k_stride = k_new_stride;
  append.v_new = v_new;
  append.v_stride = v_new_stride;
  append.cos_table = cos_table;
  append.sin_table = sin_table;
  append.table_rows = table_rows;
  return paged_decode_call(dtype, q, q_stride_b, q_stride_h, k_cache, v_cache, num_layers, layer_index, num_blocks,
                           block_size, q_heads, kv_heads, head_dim, block_tables, table_stride, seq_lens, batch,
                           max_seq_len, total_seq_len, scale, out, out_stride_b, out_stride_h, workspace,
                           workspace_bytes, host_seq_lens, append, stream);
}

NIE_API int64_t nie_paged_decode_plan_bytes(void) { return (int64_t)sizeof(DecodeItems); }

NIE_API int nie_paged_decode_plan(int dtype, int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                  int64_t block_size, const int32_t* host_seq_lens, int64_t batch,
                                  int64_t max_seq_len, int64_t total_seq_len, void* plan, int64_t plan_bytes) {
  int rc = check_dtype(dtype);
  if (rc) return rc;
  rc = check_attention_shape(q_heads, kv_heads, head_dim, 1, block_size);
  if (rc) return rc;
  if (block_size <= 0) return fail(NIE_EINVAL, "block_size must be positive");
  if (plan == nullptr || plan_bytes < (int64_t)sizeof(DecodeItems) || ((uintptr_t)plan % alignof(DecodeItems))) {
    return fail(NIE_EINVAL, "plan buffer must hold nie_paged_decode_plan_bytes() aligned bytes");
  }
  DecodeItems* out = reinterpret_cast<DecodeItems*>(plan);
  out->count = 0;
  out->tps = 0;
  if (batch < 0) return fail(NIE_EINVAL, "batch must be non-negative");
  if (batch == 0 || !tuned_attention(head_dim, q_heads, kv_heads)) return NIE_OK;  // nothing to plan
  if (host_seq_lens == nullptr || !host_lens_ok(host_seq_lens, batch, max_seq_len, total_seq_len)) {
    return fail(NIE_EINVAL, "host lengths must be in [1, max_seq_len], reach max_seq_len and sum to total_seq_len");
  }
  fill_decode_items(plan_decode(dtype, head_dim, kv_heads, block_size, batch, total_seq_len, host_seq_lens),
                    host_seq_lens, batch, out);
  // a plan the table cannot hold: the launch plans from its bounds (a caller
  // that wants the same results eagerly plans from bounds too)
  if (out->count == 0) out->tps = 0;
  return NIE_OK;
}

NIE_API int nie_paged_decode_append_planned(int dtype, const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                            const void* k_new, int64_t k_new_stride, const void* v_new,
                                            int64_t v_new_stride, const void* cos_table, const void* sin_table,
                                            int64_t table_rows, void* k_cache, void* v_cache, int64_t num_layers,
                                            int64_t layer_index, int64_t num_blocks, int64_t block_size,
                                            int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                            const int32_t* block_tables, int64_t table_stride,
                                            const int32_t* seq_lens, int64_t batch, int64_t max_seq_len,
                                            int64_t total_seq_len, float scale, void* out, int64_t out_stride_b,
                                            int64_t out_stride_h, void* workspace, int64_t workspace_bytes,
                                            const void* device_plan, void* stream) {
  if (batch > 0 && (!k_new || !v_new)) return fail(NIE_EINVAL, "null pointer argument");
  if (device_plan == nullptr || ((uintptr_t)device_plan % alignof(DecodeItems))) {
    return fail(NIE_EINVAL, "device_plan must be an aligned device buffer of nie_paged_decode_plan_bytes() bytes");
  }
  DecodeAppend append;
  append.k_new = k_new;
  append.k_stride = k_new_stride;
  append.v_new = v_new;
  append.v_stride = v_new_stride;
  append.cos_table = cos_table;
  append.sin_table = sin_table;
  append.table_rows = table_rows;
  return paged_decode_call(dtype, q, q_stride_b, q_stride_h, k_cache, v_cache, num_layers, layer_index, num_blocks,
                           block_size, q_heads, kv_heads, head_dim, block_tables, table_stride, seq_lens, batch,
                           max_seq_len, total_seq_len, scale, out, out_stride_b, out_stride_h, workspace,
                           workspace_bytes, nullptr, append, stream, /*static_scratch=*/false, device_plan);
}

// ---------------------------------------------------------------------------
// Allocation-free decode step.  The split partials of
// nie_paged_decode_append_noalloc live in `scratch`, a library-owned device
// array (each GPU that loads the library holds its own copy, at its own
// address, until the process ends).  In host code `scratch` names a host
// stand-in, not device memory, so host code never passes it to a kernel:
// the device address is looked up once per device with hipGetSymbolAddress
// (with that device current) and kept in g_scratch_ptr.  The partials are
// fully written by the decode kernel before the merge kernel reads them, so
// the array needs no clearing between calls; calls that overlap in time on
// one GPU share it and race.
// ---------------------------------------------------------------------------
constexpr int64_t kScratchBytes = 32ll << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kScratchDevices] = {};

// Device address of `scratch` on the device that owns `stream` (the current
// device for the null stream).
int scratch_address(void* stream, void** out) {
  int dev = -1;
  hipError_t err = hipStreamGetDevice((hipStream_t)stream, &dev);
  if (err != hipSuccess) return fail(NIE_EINVAL, "hipStreamGetDevice failed: %s", hipGetErrorString(err));
  if (dev < 0 || dev >= kScratchDevices) {
    return fail(NIE_EUNSUPPORTED, "device %d is beyond the %d devices the static scratch tracks", dev,
                kScratchDevices);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    int cur = -1;
    err = hipGetDevice(&cur);
    if (err != hipSuccess) return fail(NIE_ELAUNCH, "hipGetDevice failed: %s", hipGetErrorString(err));
    if (cur != dev && (err = hipSetDevice(dev)) != hipSuccess) {
      return fail(NIE_ELAUNCH, "hipSetDevice(%d) failed: %s", dev, hipGetErrorString(err));
    }
    void* p = nullptr;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (err != hipSuccess || p == nullptr) {
      return fail(NIE_ELAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                  hipGetErrorString(err));
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return NIE_OK;
}

}  // namespace

NIE_API int64_t nie_paged_decode_noalloc_max_bytes(void) { return kScratchBytes; }

NIE_API int nie_paged_decode_append_noalloc(int dtype, const void* q, int64_t q_stride_b, int64_t q_stride_h,
                                            const void* k_new, int64_t k_new_stride, const void* v_new,
                                            int64_t v_new_stride, const void* cos_table, const void* sin_table,
                                            int64_t table_rows, void* k_cache, void* v_cache, int64_t num_layers,
                                            int64_t layer_index, int64_t num_blocks, int64_t block_size,
                                            int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                                            const int32_t* block_tables, int64_t table_stride,
                                            const int32_t* seq_lens, int64_t batch, int64_t max_seq_len,
                                            int64_t total_seq_len, float scale, void* out, int64_t out_stride_b,
                                            int64_t out_stride_h, const int32_t* host_seq_lens, void* stream) {
  if (batch > 0 && (!k_new || !v_new)) return fail(NIE_EINVAL, "null pointer argument");
  void* ws = nullptr;
  if (batch > 0) {
    const int rc = scratch_address(stream, &ws);
    if (rc) return rc;
  }
  DecodeAppend append;
  append.k_new = k_new;
  append.k_stride = k_new_stride;
  append.v_new = v_new;
  append.v_stride = v_new_stride;
  append.cos_table = cos_table;
  append.sin_table = sin_table;
  append.table_rows = table_rows;
  return paged_decode_call(dtype, q, q_stride_b, q_stride_h, k_cache, v_cache, num_layers, layer_index, num_blocks,
                           block_size, q_heads, kv_heads, head_dim, block_tables, table_stride, seq_lens, batch,
                           max_seq_len, total_seq_len, scale, out, out_stride_b, out_stride_h, ws, kScratchBytes,
                           host_seq_lens, append, stream, /*static_scratch=*/true);
}

NIE_API int64_t nie_varlen_prefill_workspace_bytes(int64_t num_seqs, int64_t total_query_tokens,
                                                   int64_t max_query_len, int64_t max_seq_len,
                                                   int64_t q_heads, int64_t kv_heads,
                                                   int64_t head_dim, const int64_t* host_cu_seqlens,
                                                   const int32_t* host_context_lens) {
  if (num_seqs <= 0 || total_query_tokens <= 0 || max_seq_len <= 0 || max_query_len <= 0 ||
      check_attention_shape(q_heads, kv_heads, head_dim, 1, 1) != NIE_OK) {
    return 0;
  }
  const bool host = host_cu_seqlens != nullptr && host_context_lens != nullptr;
  if (host && !host_metadata_ok(host_cu_seqlens, host_context_lens, num_seqs, total_query_tokens, max_query_len,
                                max_seq_len)) {
    return 0;
  }
  if (!tuned_attention(head_dim, q_heads, kv_heads)) return 0;  // the generic kernel needs no workspace
  const PrefillPlan p = plan_prefill(q_heads / kv_heads, kv_heads, num_seqs, total_query_tokens, max_seq_len,
                                     host ? host_cu_seqlens : nullptr, host ? host_context_lens : nullptr);
  // no query tile is split and, with the one-pass rounding, no (max, sum)
  // slots are needed (the query has no dtype: with the reference rounding it
  // sizes for bf16, which an fp32 call can use too)
  if (!p.split && g_rounding.load(std::memory_order_relaxed) != NIE_ROUND_REFERENCE) return 0;
  return kCtlBytes + p.items * kv_heads * p.rows * (head_dim + 4) * (int64_t)sizeof(float);
}

NIE_API int nie_varlen_prefill(int dtype, const void* q, int64_t q_stride_t, int64_t q_stride_h,
                               const int64_t* cu_seqlens_q, const int32_t* context_lens,
                               int64_t num_seqs, int64_t total_query_tokens,
                               int64_t max_query_len, int64_t max_seq_len, const void* k_cache,
                               const void* v_cache, int64_t num_layers, int64_t layer_index,
                               int64_t num_blocks, int64_t block_size, int64_t q_heads,
                               int64_t kv_heads, int64_t head_dim, const int32_t* block_tables,
                               int64_t table_stride, float scale, void* out,
                               int64_t out_stride_t, int64_t out_stride_h, void* workspace,
                               int64_t workspace_bytes, const int64_t* host_cu_seqlens,
                               const int32_t* host_context_lens, void* stream) {
  int rc = check_dtype(dtype);
  if (rc) return rc;
  rc = check_geometry(num_layers, layer_index, num_blocks, block_size, kv_heads, head_dim);
  if (rc) return rc;
  rc = check_attention_shape(q_heads, kv_heads, head_dim, num_blocks, block_size);
  if (rc) return rc;
  if (num_seqs < 0 || total_query_tokens < 0) return fail(NIE_EINVAL, "negative sizes");
  if (num_seqs == 0 || total_query_tokens == 0) return NIE_OK;
  if (!q || !cu_seqlens_q || !context_lens || !k_cache || !v_cache || !block_tables || !out) {
    return fail(NIE_EINVAL, "null pointer argument");
  }
  if (max_query_len <= 0 || max_query_len > total_query_tokens || max_seq_len < max_query_len ||
      max_seq_len > 0x7fffffffLL - kTileKeys) {
    return fail(NIE_EINVAL, "inconsistent max_query_len / max_seq_len");
  }
  if (table_stride <= 0 || table_stride > 0x7fffffffLL || table_stride * block_size < max_seq_len) {
    return fail(NIE_EINVAL, "block table row does not cover max_seq_len");
  }
  const int64_t es = elt_bytes(dtype);
  if (!tuned_attention(head_dim, q_heads, kv_heads)) {
    // other shapes: the generic kernel (no workspace; element alignment)
    if (!elt_aligned(es, {q, out, k_cache, v_cache})) return fail(NIE_EINVAL, "pointers must be aligned to the element size");
    GenericAttnArgs ga{};
    ga.q = q;
    ga.q_sr = q_stride_t;
    ga.q_sh = q_stride_h;
    ga.out = out;
    ga.o_sr = out_stride_t;
    ga.o_sh = out_stride_h;
    ga.k_cache = k_cache;
    ga.v_cache = v_cache;
    ga.geom = make_geom(layer_index, num_blocks, block_size, kv_heads, head_dim);
    ga.head_dim = (int32_t)head_dim;
    ga.q_heads = (int32_t)q_heads;
    ga.group = (int32_t)(q_heads / kv_heads);
    ga.tables = block_tables;
    ga.table_stride = table_stride;
    ga.scale = scale;
    ga.rows = total_query_tokens;
    ga.cu_seqlens = cu_seqlens_q;
    ga.context_lens = context_lens;
    ga.num_seqs = num_seqs;
    return generic_attention(dtype, ga, (hipStream_t)stream);
  }
  if (!check_aligned(q, q_stride_t, q_stride_h, es) || !check_aligned(out, out_stride_t, out_stride_h, es) ||
      ((uintptr_t)k_cache % 16) || ((uintptr_t)v_cache % 16)) {
    return fail(NIE_EINVAL, "q/out/cache pointers and strides must be 16-byte aligned");
  }
  const bool host = host_cu_seqlens != nullptr && host_context_lens != nullptr;
  if (host && !host_metadata_ok(host_cu_seqlens, host_context_lens, num_seqs, total_query_tokens, max_query_len,
                                max_seq_len)) {
    return fail(NIE_EINVAL, "host cu_seqlens / context_lens do not match the sizes of the call");
  }
  const int group = (int)(q_heads / kv_heads);
  const PrefillPlan plan = plan_prefill(group, kv_heads, num_seqs, total_query_tokens, max_seq_len,
                                        host ? host_cu_seqlens : nullptr, host ? host_context_lens : nullptr);
  // 1-D grids: items x heads prefill workgroups, tiles x heads x row groups merge workgroups
  if (plan.items * kv_heads > 0xffffffffLL / (kPrefillWaves * kWave) ||
      plan.qtiles * kv_heads * (plan.rows / kPrefillMergeRows) > 0xffffffffLL / (kPrefillMergeWaves * kWave) ||
      total_query_tokens > 0x7fffffffLL) {
    return fail(NIE_EINVAL, "grid too large");
  }
  if (plan.items == 0) return NIE_OK;
  const bool may_split = plan.split;
  // the reference rounding always needs the workspace: every item's
  // (max, sum) slots, one piece included
  const bool two = two_pass(dtype);
  // the workspace: the control region (which prefill leaves alone), then
  // the partials
  // the control region, the partials, then two (max, sum) slots per item
  // and row (the stats pass's parts)
  const int64_t need = kCtlBytes + plan.items * kv_heads * plan.rows * (head_dim + 4) * (int64_t)sizeof(float);
  if ((may_split || two) && (workspace == nullptr || workspace_bytes < need || ((uintptr_t)workspace % 16))) {
    return fail(NIE_EINVAL, "workspace too small: need %lld bytes, got %lld", (long long)need,
                (long long)workspace_bytes);
  }
  PrefillArgs a;
  a.q = q;
  a.q_st = q_stride_t;
  a.q_sh = q_stride_h;
  a.cu_seqlens = cu_seqlens_q;
  a.context_lens = context_lens;
  a.num_seqs = num_seqs;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.geom = make_geom(layer_index, num_blocks, block_size, kv_heads, head_dim);
  a.group = group;
  a.tokens_per_tile = plan.tokens_per_tile;
  a.tiles_per_split = (int32_t)plan.tps;
  a.grid_items = (int32_t)plan.items;
  a.merge_tiles = 0;
  a.tables = block_tables;
  a.table_stride = table_stride;
  a.scale = scale;
  a.out = out;
  a.o_st = out_stride_t;
  a.o_sh = out_stride_h;
  const bool have_ws = (may_split || two) && workspace != nullptr && workspace_bytes >= need;
  a.ws_o = have_ws ? reinterpret_cast<float*>(reinterpret_cast<unsigned char*>(workspace) + kCtlBytes) : nullptr;
  a.ws_ml = have_ws ? a.ws_o + plan.items * kv_heads * plan.rows * head_dim : nullptr;
  a.ws_items = have_ws ? plan.items : 0;
  a.ws_ml_slots = have_ws ? 2 * plan.items : 0;
  // parts of two in the stats pass when its workgroups would otherwise
  // leave room on the CUs (it holds four per CU, the other passes two)
  a.stats_parts = two && plan.items * kv_heads <= 2 * device_cus() ? 2 : 1;
  PrefillMergeJobs jobs;
  jobs.count = 0;
  if (may_split) fill_merge_jobs(plan, num_seqs, host ? host_cu_seqlens : nullptr, host ? host_context_lens : nullptr, &jobs);
  PrefillSchedule sched;
  if (host) build_prefill_schedule(plan, num_seqs, host_cu_seqlens, host_context_lens, &sched);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == NIE_DTYPE_BF16) {
    if (head_dim == 64) launch_prefill<bf16_t, 64>(a, plan, sched, jobs, s, may_split, two);
    else launch_prefill<bf16_t, 128>(a, plan, sched, jobs, s, may_split, two);
  } else {
    if (head_dim == 64) launch_prefill<float, 64>(a, plan, sched, jobs, s, may_split, false);
    else launch_prefill<float, 128>(a, plan, sched, jobs, s, may_split, false);
  }
  return launched("varlen_prefill");
}
