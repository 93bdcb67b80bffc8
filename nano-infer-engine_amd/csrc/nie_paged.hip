// nie_paged.hip — paged-attention kernels for MI355X (gfx950 / CDNA4).
//
// Kernels
//   kv_append_kernel        slot-mapped scatter of new K/V rows into the cache
//   kv_gather_kernel        logical -> contiguous copy of one sequence
//   kv_copy_blocks_kernel   whole-block copies (export / import of sequences)
//   paged_decode_kernel     split-K decode attention, one workgroup per
//                           (sequence, key-split), one wave per KV head
//   decode_merge_kernel     exact fp32 merge of the split-K partials
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

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>

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

// float -> bf16, round to nearest even (torch's conversion).  NaN stays NaN.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float x) {
  uint32_t u = __float_as_uint(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ float round_to_bf16(float x) {
  return bf16_bits_to_f32(f32_to_bf16_bits(x));
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
// (lanes l, l^16, l^32, l^48).
__device__ __forceinline__ float sum_over_groups(float x) {
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

__device__ __forceinline__ float max_over_groups(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  x = fmaxf(x, __shfl_xor(x, 32));
  return x;
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
      *seq = b0 + src;
      *first = base + __shfl(excl, src);
      *count = __shfl(n, src);
      *local = item - *first;
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

// Addressing of the 16 keys of one tile (tiles start at multiples of 16).
// kUniform: block_size is a multiple of 16, so the whole tile lies in one
// physical block and a single (scalar) table lookup serves all lanes.
template <bool kUniform>
struct TileAddr {
  int64_t base;
  __device__ __forceinline__ void init(const CacheGeom& g, const int32_t* table, int table_len,
                                       int key0) {
    if constexpr (kUniform) base = token_offset(g, table, table_len, key0);
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

template <int N>
__device__ __forceinline__ void load_vecs(uint4 (&dst)[N], const void* src) {
  const uint4* s = reinterpret_cast<const uint4*>(src);
#pragma unroll
  for (int i = 0; i < N; ++i) dst[i] = s[i];
}

// ---------------------------------------------------------------------------
// MFMA tile math shared by decode and prefill
// ---------------------------------------------------------------------------
// Each lane holds, for its row (l%16: the key for K, the query row for Q),
// the D/4 consecutive dims starting at (D/4)*(l/16).  The MFMA K index is
// mapped onto those dims identically for both operands, so the sum over all
// MFMAs is the full q.k dot product.
template <typename T, int D>
struct Frag {
  static constexpr int kBytes = D * Elt<T>::kBytes / 4;  // bytes of one lane's slice
  static constexpr int kVec = kBytes / 16;               // 16-byte vectors per slice
  uint4 v[kVec];
};

template <typename T, int D>
__device__ __forceinline__ v4f qk_mfma(const Frag<T, D>& k, const Frag<T, D>& q) {
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  if constexpr (Elt<T>::kIsBf16) {
    const uint32_t* kw = reinterpret_cast<const uint32_t*>(k.v);
    const uint32_t* qw = reinterpret_cast<const uint32_t*>(q.v);
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      v4s a, b;
      a[0] = (short)(kw[2 * c] & 0xffff);
      a[1] = (short)(kw[2 * c] >> 16);
      a[2] = (short)(kw[2 * c + 1] & 0xffff);
      a[3] = (short)(kw[2 * c + 1] >> 16);
      b[0] = (short)(qw[2 * c] & 0xffff);
      b[1] = (short)(qw[2 * c] >> 16);
      b[2] = (short)(qw[2 * c + 1] & 0xffff);
      b[3] = (short)(qw[2 * c + 1] >> 16);
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
  float tmax = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
  tmax = max_over_groups(tmax);
  const float m_new = fmaxf(st.m, tmax);
  // A row with nothing unmasked so far keeps m = -inf; use 0 as the
  // reference point so the exponentials below are exact zeros, not NaN.
  const float ref = (m_new == kNegInf) ? 0.f : m_new;
  const float alpha = exp2f((st.m - ref) * kLog2e);
  float tsum = 0.f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s[i] = exp2f((s[i] - ref) * kLog2e);
    tsum += s[i];
  }
  st.lsum = st.lsum * alpha + tsum;
  st.m = m_new;
#pragma unroll
  for (int c = 0; c < D / 16; ++c) st.o[c] *= alpha;
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
    v4s b;
#pragma unroll
    for (int i = 0; i < 4; ++i) b[i] = (short)f32_to_bf16_bits(p[i]);
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
    w.x = f32_to_bf16_bits(a) | (f32_to_bf16_bits(b) << 16);
    w.y = f32_to_bf16_bits(c) | (f32_to_bf16_bits(d) << 16);
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
// Paged decode (split-K)
// ---------------------------------------------------------------------------
constexpr int kDecodeWaves = 8;  // KV heads handled by one workgroup (one per wave)

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
  int32_t tiles_per_split;  // 16-key tiles per work item
  float scale;
  void* out;
  int64_t o_sb, o_sh;
  float* ws_o;   // (ws_items, q_heads, head_dim)
  float* ws_ml;  // (ws_items, q_heads, 2)
  int64_t ws_items;  // partial slots in the workspace (0 when there is none)
};

__device__ __forceinline__ int64_t decode_splits_of(const DecodeArgs& a, int64_t b) {
  const int64_t len = a.seq_lens[b];
  return len > 0 ? cdiv(cdiv(len, kTileKeys), a.tiles_per_split) : (int64_t)0;
}

template <typename T, int D, bool kUniform>
__global__ __launch_bounds__(kDecodeWaves* kWave) void paged_decode_kernel(DecodeArgs a) {
  constexpr int kRowBytes = D * Elt<T>::kBytes;
  constexpr int kPitch = kRowBytes + kLdsPadBytes;
  constexpr int kChunksPerRow = kRowBytes / 16;        // 16-byte chunks per V row
  constexpr int kRowsPerPass = kWave / kChunksPerRow;  // V rows one load instruction covers
  constexpr int kPasses = kTileKeys / kRowsPerPass;    // load instructions per V tile
  constexpr int kEltPerChunk = 16 / Elt<T>::kBytes;
  using F = Frag<T, D>;
  __shared__ __attribute__((aligned(16))) unsigned char lds[kDecodeWaves][kTileKeys * kPitch];

  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int g = lane >> 4;
  const int row = lane & 15;

  int64_t b, split, first_item, nsplit;
  locate_item((int64_t)blockIdx.x, a.batch, [&](int64_t s) { return decode_splits_of(a, s); },
              &b, &split, &first_item, &nsplit);
  if (b < 0) return;
  const int h = (int)blockIdx.y * kDecodeWaves + wave;
  if (h >= a.geom.kv_heads) return;

  const int seq_len = a.seq_lens[b];
  const int32_t* table = a.tables + b * a.table_stride;
  const int tlen = (int)a.table_stride;
  const int key_begin = (int)split * a.tiles_per_split * kTileKeys;
  const int key_end = min(key_begin + a.tiles_per_split * kTileKeys, seq_len);
  const int last = key_end - 1;

  // Lane-specific base pointers: this lane's K slice and V chunk of head h.
  const T* kc = reinterpret_cast<const T*>(a.k_cache) + h * D + g * (D / 4);
  const T* vc = reinterpret_cast<const T*>(a.v_cache) + h * D + (lane % kChunksPerRow) * kEltPerChunk;

  // Q^T operand: row -> query head h*group + row (rows >= group are zero).
  F qf;
  const bool row_valid = row < a.group;
  const int qh = h * a.group + row;
  if (row_valid) {
    load_vecs(qf.v, reinterpret_cast<const T*>(a.q) + b * a.q_sb + qh * a.q_sh + g * (D / 4));
  } else {
#pragma unroll
    for (int i = 0; i < F::kVec; ++i) qf.v[i] = uint4{0u, 0u, 0u, 0u};
  }

  SoftmaxState<D> st;
  st.init();
  unsigned char* vt = lds[wave];

  // Register double buffer of whole tiles (K slice = A operand, V chunks).
  // Tiles are passed by value and every prefetch is unconditional (past the
  // end it re-reads the split's last tile, an L2 hit), which keeps both
  // buffers in VGPRs.  Keys past the end of the sequence are clamped to the
  // last valid key, so no lane reads a slot the sequence does not own; those
  // keys are masked to p = 0.
  struct Tile {
    F k;
    uint4 v[kPasses];
  };
  auto fetch = [&](int key0) {
    Tile tl;
    TileAddr<kUniform> ta;
    ta.init(a.geom, table, tlen, key0);
    const int lim = last - key0;
    load_vecs(tl.k.v, kc + ta.at(a.geom, table, tlen, key0, min(row, lim)));
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int r = min(p * kRowsPerPass + lane / kChunksPerRow, lim);
      tl.v[p] = *reinterpret_cast<const uint4*>(vc + ta.at(a.geom, table, tlen, key0, r));
    }
    return tl;
  };
  auto consume = [&](const Tile& tl, int key0) {
    // Stage V into this wave's LDS rows ([key][dim]) for the transposed read.
#pragma unroll
    for (int p = 0; p < kPasses; ++p) {
      const int r = p * kRowsPerPass + lane / kChunksPerRow;
      *reinterpret_cast<uint4*>(vt + r * kPitch + (lane % kChunksPerRow) * 16) = tl.v[p];
    }
    v4f s = qk_mfma<T, D>(tl.k, qf);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s[i] = (key0 + 4 * g + i <= last) ? scaled_score<T>(s[i], a.scale) : kNegInf;
    }
    softmax_tile<D>(st, s);
    pv_mfma<T, D>(st, vt, kPitch, s);
  };

  const int ntiles = (key_end - key_begin + kTileKeys - 1) / kTileKeys;
  const int last_key0 = key_begin + (ntiles - 1) * kTileKeys;
  Tile t0 = fetch(key_begin);
  for (int t = 0; t < ntiles; t += 2) {
    const int key0 = key_begin + t * kTileKeys;
    const Tile t1 = fetch(min(key0 + kTileKeys, last_key0));
    consume(t0, key0);
    if (t + 1 >= ntiles) break;
    t0 = fetch(min(key0 + 2 * kTileKeys, last_key0));
    consume(t1, key0 + kTileKeys);
  }

  const float lsum = sum_over_groups(st.lsum);
  if (!row_valid) return;
  if (nsplit == 1) {
    const float inv = 1.f / lsum;
    T* dst = reinterpret_cast<T*>(a.out) + b * a.o_sb + qh * a.o_sh + 4 * g;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      store4<T>(dst + 16 * c, st.o[c][0] * inv, st.o[c][1] * inv, st.o[c][2] * inv,
                st.o[c][3] * inv);
    }
  } else {
    const int64_t item = first_item + split;
    // Only reachable with a workspace; the bound keeps inconsistent length
    // hints from writing outside it.
    if (a.ws_o == nullptr || item >= a.ws_items) return;
    float* dst = a.ws_o + (item * a.q_heads + qh) * D + 4 * g;
#pragma unroll
    for (int c = 0; c < D / 16; ++c) {
      *reinterpret_cast<float4*>(dst + 16 * c) = make_float4(st.o[c][0], st.o[c][1], st.o[c][2], st.o[c][3]);
    }
    if (g == 0) {
      float* ml = a.ws_ml + (item * a.q_heads + qh) * 2;
      ml[0] = st.m;
      ml[1] = lsum;
    }
  }
}

// grid (batch, ceil(q_heads/4)), 4 waves: one wave per (sequence, query
// head) merges that row's split partials in fp32.
template <typename T, int D>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeArgs a) {
  const int lane = lane_id();
  const int64_t b = blockIdx.x;
  const int qh = (int)blockIdx.y * 4 + (int)(threadIdx.x / kWave);
  if (b >= a.batch) return;
  // first item of sequence b = number of items of the sequences before it
  int64_t first = 0;
  for (int64_t b0 = 0; b0 < b; b0 += kWave) {
    const int64_t s = b0 + lane;
    int64_t n = (s < b) ? decode_splits_of(a, s) : 0;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) n += __shfl_xor(n, off);
    first += n;
  }
  const int64_t nsplit = decode_splits_of(a, b);
  if (qh >= a.q_heads || nsplit <= 1 || a.ws_o == nullptr || first + nsplit > a.ws_items) return;
  float mmax = kNegInf;
  for (int64_t s = 0; s < nsplit; ++s) {
    mmax = fmaxf(mmax, a.ws_ml[((first + s) * a.q_heads + qh) * 2]);
  }
  constexpr int kPerLane = D / kWave;
  float denom = 0.f;
  float acc[kPerLane];
#pragma unroll
  for (int j = 0; j < kPerLane; ++j) acc[j] = 0.f;
  for (int64_t s = 0; s < nsplit; ++s) {
    const int64_t idx = (first + s) * a.q_heads + qh;
    const float m = a.ws_ml[idx * 2];
    const float w = (m == kNegInf) ? 0.f : exp2f((m - mmax) * kLog2e);
    denom += w * a.ws_ml[idx * 2 + 1];
#pragma unroll
    for (int j = 0; j < kPerLane; ++j) acc[j] += w * a.ws_o[idx * D + j * kWave + lane];
  }
  const float inv = 1.f / denom;
  T* dst = reinterpret_cast<T*>(a.out) + b * a.o_sb + qh * a.o_sh;
#pragma unroll
  for (int j = 0; j < kPerLane; ++j) store_elt<T>(dst + j * kWave + lane, acc[j] * inv);
}

// Work decomposition of a decode call: 16-key tiles per split chosen so the
// batch yields about kDecodeTargetItems workgroups per group of 8 KV heads
// (two resident workgroups on each of the 256 CUs).
constexpr int64_t kDecodeTargetItems = 512;
constexpr int64_t kDecodeMinTilesPerSplit = 4;

int64_t decode_tiles_per_split(int64_t batch, int64_t total_seq_len) {
  const int64_t total_tiles = cdiv(total_seq_len, kTileKeys) + batch;
  const int64_t tps = cdiv(total_tiles, kDecodeTargetItems);
  return tps < kDecodeMinTilesPerSplit ? kDecodeMinTilesPerSplit : tps;
}

int64_t decode_max_items(int64_t batch, int64_t total_seq_len, int64_t tps) {
  // sum_b ceil(ceil(len_b/16)/tps) <= (sum_b len_b/16 + batch)/tps + batch
  return (cdiv(total_seq_len, kTileKeys) + batch) / tps + batch + 1;
}

// ---------------------------------------------------------------------------
// Varlen prefill
// ---------------------------------------------------------------------------
constexpr int kPrefillWaves = 4;

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
  int32_t tokens_per_tile;  // query tokens per workgroup
  const int32_t* tables;
  int64_t table_stride;
  float scale;
  void* out;
  int64_t o_st, o_sh;
};

template <typename T, int D, bool kUniform>
__global__ __launch_bounds__(kPrefillWaves* kWave) void varlen_prefill_kernel(PrefillArgs a) {
  constexpr int kRowBytes = D * Elt<T>::kBytes;
  constexpr int kPitch = kRowBytes + kLdsPadBytes;
  constexpr int kChunksPerRow = kRowBytes / 16;
  constexpr int kChunksPerTile = kTileKeys * kChunksPerRow;  // per K (or V) tile
  constexpr int kThreads = kPrefillWaves * kWave;
  constexpr int kLoadsPerThread = (2 * kChunksPerTile) / kThreads;  // K and V together
  constexpr int kEltPerChunk = 16 / Elt<T>::kBytes;
  static_assert((2 * kChunksPerTile) % kThreads == 0, "tile chunks must divide evenly");
  using F = Frag<T, D>;
  __shared__ __attribute__((aligned(16))) unsigned char k_lds[kTileKeys * kPitch];
  __shared__ __attribute__((aligned(16))) unsigned char v_lds[kTileKeys * kPitch];

  const int lane = lane_id();
  const int wave = threadIdx.x / kWave;
  const int g = lane >> 4;
  const int row = lane & 15;
  const int tpt = a.tokens_per_tile;

  int64_t r, tile, first_tile, ntile_r;
  locate_item(
      (int64_t)blockIdx.x, a.num_seqs,
      [&](int64_t s) { return cdiv(a.cu_seqlens[s + 1] - a.cu_seqlens[s], (int64_t)tpt); },
      &r, &tile, &first_tile, &ntile_r);
  if (r < 0) return;  // same for every wave of the workgroup
  const int h = (int)blockIdx.y;

  const int64_t q_begin = a.cu_seqlens[r];
  const int q_len = (int)(a.cu_seqlens[r + 1] - q_begin);
  const int ctx = a.context_lens[r];
  const int32_t* table = a.tables + r * a.table_stride;
  const int tlen = (int)a.table_stride;
  const int t0 = (int)tile * tpt;                  // first query token of the tile
  const int t_end = min(t0 + tpt, q_len);
  const int key_end = ctx + t_end;                 // keys visible to the tile's last row

  // This lane's query row: token t0 + wave*(16/group) + row/group, head row%group.
  const int tokens_per_wave = 16 / a.group;
  const int tq = t0 + wave * tokens_per_wave + row / a.group;
  const int qh = h * a.group + row % a.group;
  const bool row_valid = tq < t_end;
  const int q_pos = ctx + tq;

  F qf;
  if (row_valid) {
    load_vecs(qf.v, reinterpret_cast<const T*>(a.q) + (q_begin + tq) * a.q_st + qh * a.q_sh + g * (D / 4));
  } else {
#pragma unroll
    for (int i = 0; i < F::kVec; ++i) qf.v[i] = uint4{0u, 0u, 0u, 0u};
  }

  const T* kc = reinterpret_cast<const T*>(a.k_cache) + h * D;
  const T* vc = reinterpret_cast<const T*>(a.v_cache) + h * D;

  uint4 stage[kLoadsPerThread];
  auto fetch = [&](int key0) {
    TileAddr<kUniform> ta;
    ta.init(a.geom, table, tlen, key0);
    const int lim = key_end - 1 - key0;
#pragma unroll
    for (int j = 0; j < kLoadsPerThread; ++j) {
      const int chunk = threadIdx.x + j * kThreads;  // 0 .. 2*kChunksPerTile-1
      const int c = chunk % kChunksPerTile;
      const int rr = min(c / kChunksPerRow, lim);
      const T* base = (chunk < kChunksPerTile) ? kc : vc;
      stage[j] = *reinterpret_cast<const uint4*>(base + ta.at(a.geom, table, tlen, key0, rr) +
                                                 (c % kChunksPerRow) * kEltPerChunk);
    }
  };
  auto commit = [&]() {
#pragma unroll
    for (int j = 0; j < kLoadsPerThread; ++j) {
      const int chunk = threadIdx.x + j * kThreads;
      const int c = chunk % kChunksPerTile;
      unsigned char* dst = (chunk < kChunksPerTile ? k_lds : v_lds) + (c / kChunksPerRow) * kPitch +
                           (c % kChunksPerRow) * 16;
      *reinterpret_cast<uint4*>(dst) = stage[j];
    }
  };

  SoftmaxState<D> st;
  st.init();
  const int ntiles = (key_end + kTileKeys - 1) / kTileKeys;
  fetch(0);
  for (int t = 0; t < ntiles; ++t) {
    const int key0 = t * kTileKeys;
    __syncthreads();  // every wave is done with the previous tile
    commit();
    __syncthreads();
    fetch(min(key0 + kTileKeys, (ntiles - 1) * kTileKeys));  // past the end: re-read (L2 hit)
    F kf;
    load_vecs(kf.v, k_lds + row * kPitch + g * F::kBytes);
    v4f s = qk_mfma<T, D>(kf, qf);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // S^T C-layout: this value is key key0 + 4g + i of this lane's row.
      const int key = key0 + 4 * g + i;
      s[i] = (key <= q_pos && key < key_end) ? scaled_score<T>(s[i], a.scale) : kNegInf;
    }
    softmax_tile<D>(st, s);
    pv_mfma<T, D>(st, v_lds, kPitch, s);
  }

  const float lsum = sum_over_groups(st.lsum);
  if (!row_valid) return;
  const float inv = 1.f / lsum;
  T* dst = reinterpret_cast<T*>(a.out) + (q_begin + tq) * a.o_st + qh * a.o_sh + 4 * g;
#pragma unroll
  for (int c = 0; c < D / 16; ++c) {
    store4<T>(dst + 16 * c, st.o[c][0] * inv, st.o[c][1] * inv, st.o[c][2] * inv,
              st.o[c][3] * inv);
  }
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

int check_attention_shape(int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                          int64_t num_blocks, int64_t block_size) {
  if (head_dim != 64 && head_dim != 128) {
    return fail(NIE_EUNSUPPORTED, "head_dim %lld not supported (64 or 128)", (long long)head_dim);
  }
  if (q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads != 0) {
    return fail(NIE_EINVAL, "q_heads (%lld) must be a positive multiple of kv_heads (%lld)",
                (long long)q_heads, (long long)kv_heads);
  }
  const int64_t group = q_heads / kv_heads;
  if (group != 1 && group != 2 && group != 4 && group != 8 && group != 16) {
    return fail(NIE_EUNSUPPORTED, "GQA group size %lld not supported", (long long)group);
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

template <typename T, int D, bool U>
void launch_decode_t(const DecodeArgs& a, int64_t items, hipStream_t stream, bool merge) {
  const dim3 grid((unsigned)items, (unsigned)cdiv(a.geom.kv_heads, kDecodeWaves));
  const int waves = a.geom.kv_heads < kDecodeWaves ? a.geom.kv_heads : kDecodeWaves;
  hipLaunchKernelGGL((paged_decode_kernel<T, D, U>), grid, dim3(waves * kWave), 0, stream, a);
  if (merge) {
    const dim3 mgrid((unsigned)a.batch, (unsigned)cdiv(a.q_heads, 4));
    hipLaunchKernelGGL((decode_merge_kernel<T, D>), mgrid, dim3(256), 0, stream, a);
  }
}

template <typename T, int D>
void launch_decode(const DecodeArgs& a, int64_t items, hipStream_t stream, bool merge) {
  if (a.geom.block_size % kTileKeys == 0) launch_decode_t<T, D, true>(a, items, stream, merge);
  else launch_decode_t<T, D, false>(a, items, stream, merge);
}

template <typename T, int D>
void launch_prefill(const PrefillArgs& a, int64_t tiles, hipStream_t stream) {
  const dim3 grid((unsigned)tiles, (unsigned)a.geom.kv_heads);
  if (a.geom.block_size % kTileKeys == 0) {
    hipLaunchKernelGGL((varlen_prefill_kernel<T, D, true>), grid, dim3(kPrefillWaves * kWave), 0, stream, a);
  } else {
    hipLaunchKernelGGL((varlen_prefill_kernel<T, D, false>), grid, dim3(kPrefillWaves * kWave), 0, stream, a);
  }
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

NIE_API int64_t nie_paged_decode_workspace_bytes(int64_t batch, int64_t q_heads, int64_t head_dim,
                                                 int64_t block_size, int64_t max_seq_len,
                                                 int64_t total_seq_len) {
  (void)block_size;
  (void)max_seq_len;
  if (batch <= 0 || q_heads <= 0 || head_dim <= 0 || total_seq_len <= 0) return 0;
  const int64_t tps = decode_tiles_per_split(batch, total_seq_len);
  const int64_t items = decode_max_items(batch, total_seq_len, tps);
  return items * q_heads * (head_dim + 2) * (int64_t)sizeof(float);
}

NIE_API int nie_paged_decode(int dtype, const void* q, int64_t q_stride_b, int64_t q_stride_h,
                             const void* k_cache, const void* v_cache, int64_t num_layers,
                             int64_t layer_index, int64_t num_blocks, int64_t block_size,
                             int64_t q_heads, int64_t kv_heads, int64_t head_dim,
                             const int32_t* block_tables, int64_t table_stride,
                             const int32_t* seq_lens, int64_t batch, int64_t max_seq_len,
                             int64_t total_seq_len, float scale, void* out,
                             int64_t out_stride_b, int64_t out_stride_h, void* workspace,
                             int64_t workspace_bytes, void* stream) {
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
  if (!check_aligned(q, q_stride_b, q_stride_h, es) || !check_aligned(out, out_stride_b, out_stride_h, es) ||
      ((uintptr_t)k_cache % 16) || ((uintptr_t)v_cache % 16)) {
    return fail(NIE_EINVAL, "q/out/cache pointers and strides must be 16-byte aligned");
  }
  const int64_t tps = decode_tiles_per_split(batch, total_seq_len);
  const int64_t items = decode_max_items(batch, total_seq_len, tps);
  const bool may_split = cdiv(max_seq_len, kTileKeys) > tps;
  const int64_t need = items * q_heads * (head_dim + 2) * (int64_t)sizeof(float);
  if (may_split && (workspace == nullptr || workspace_bytes < need)) {
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
  a.scale = scale;
  a.out = out;
  a.o_sb = out_stride_b;
  a.o_sh = out_stride_h;
  const bool have_ws = workspace != nullptr && workspace_bytes >= need;
  a.ws_o = have_ws ? reinterpret_cast<float*>(workspace) : nullptr;
  a.ws_ml = have_ws ? a.ws_o + items * q_heads * head_dim : nullptr;
  a.ws_items = have_ws ? items : 0;
  // The grid is an upper bound on the item count (exact to within `batch`);
  // workgroups past the last real item return immediately.
  hipStream_t s = (hipStream_t)stream;
  if (dtype == NIE_DTYPE_BF16) {
    if (head_dim == 64) launch_decode<bf16_t, 64>(a, items, s, may_split);
    else launch_decode<bf16_t, 128>(a, items, s, may_split);
  } else {
    if (head_dim == 64) launch_decode<float, 64>(a, items, s, may_split);
    else launch_decode<float, 128>(a, items, s, may_split);
  }
  return launched("paged_decode");
}

NIE_API int64_t nie_varlen_prefill_workspace_bytes(int64_t num_seqs, int64_t total_query_tokens,
                                                   int64_t max_query_len, int64_t max_seq_len,
                                                   int64_t q_heads, int64_t kv_heads,
                                                   int64_t head_dim) {
  // The prefill kernel writes its output directly; no scratch is needed.
  (void)num_seqs;
  (void)total_query_tokens;
  (void)max_query_len;
  (void)max_seq_len;
  (void)q_heads;
  (void)kv_heads;
  (void)head_dim;
  return 0;
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
                               int64_t workspace_bytes, void* stream) {
  (void)workspace;
  (void)workspace_bytes;
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
  if (!check_aligned(q, q_stride_t, q_stride_h, es) || !check_aligned(out, out_stride_t, out_stride_h, es) ||
      ((uintptr_t)k_cache % 16) || ((uintptr_t)v_cache % 16)) {
    return fail(NIE_EINVAL, "q/out/cache pointers and strides must be 16-byte aligned");
  }
  const int group = (int)(q_heads / kv_heads);
  const int tpt = kPrefillWaves * (16 / group);
  // sum_r ceil(len_r / tpt) <= total / tpt + num_seqs
  const int64_t tiles = total_query_tokens / tpt + num_seqs;
  if (tiles > 0x7fffffffLL) return fail(NIE_EINVAL, "grid too large");
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
  a.tokens_per_tile = tpt;
  a.tables = block_tables;
  a.table_stride = table_stride;
  a.scale = scale;
  a.out = out;
  a.o_st = out_stride_t;
  a.o_sh = out_stride_h;
  hipStream_t s = (hipStream_t)stream;
  if (dtype == NIE_DTYPE_BF16) {
    if (head_dim == 64) launch_prefill<bf16_t, 64>(a, tiles, s);
    else launch_prefill<bf16_t, 128>(a, tiles, s);
  } else {
    if (head_dim == 64) launch_prefill<float, 64>(a, tiles, s);
    else launch_prefill<float, 128>(a, tiles, s);
  }
  return launched("varlen_prefill");
}
