// GQA-native prefill attention for gfx950 (MFMA, fp32 softmax).
//
// Reference semantics: the prefill branch of threadcut/attention.py:43-46 —
// SDPA of q [b, hq, L, d] against repeat_kv(k), repeat_kv(v) (each KV head
// expanded g = hq/hkv times) with the boolean attention mask, or is_causal
// when there is no mask and L == n; output transposed to [b, L, hq, d].
// Here the KV heads are never expanded: a work-group owns 128 query rows that
// are (query token, query head of the group) pairs of ONE KV head, so every
// K/V tile it stages in LDS is read once and shared by the g heads.
//
// Per 64-key tile, each wave (32 query rows) computes
//   S^T = K . Q^T   with v_mfma_f32_32x32x16: A = K rows from LDS, B = Q^T
//                   from registers; lane l then holds 16 of the 32 keys of
//                   each 32-key half for query row l%32 (the other 16 sit in
//                   lane l^32), so a row's max and sum need one lane swap;
//   O^T += V^T . P^T with P^T fed straight from those registers (fp16/bf16)
//                   and V^T read from the V rows in LDS with the
//                   transposing read (ds_read_b64_tr_b16), so P never moves
//                   between lanes.
// The online softmax runs per query row in fp32, log2 domain, as
// p = exp2(s * c - m) with c = |scale| * log2(e) (a negative scale flips the
// sign bits of Q instead). The running maximum m moves only when a tile's
// maximum exceeds it by more than a factor 2^8, so the accumulators are
// rescaled rarely. The K and V^T fragments are read from LDS ahead of the
// MFMAs that use them.
//
// Every tile is classified for the whole work-group: SKIP (no row sees any
// of its keys: not loaded), FULL (every row sees every key: no per-element
// test), CAUSAL (per-element test by the end-aligned causal rule) or MIXED
// (per-element test against the mask bytes). Without a mask the class
// follows from n and the causal diagonal; with a boolean mask it is read
// from a map that tc_prefill_mask_tiles builds in one pass over the mask,
// once per mask.
// Tiles are double-buffered and loaded straight into LDS (16-byte buffer
// loads with the LDS bit, no registers, no LDS stores): the next active
// tile's loads are in flight while the current one is multiplied.
#include <algorithm>
#include <cmath>

#include "tc_common.hpp"

namespace tc {
namespace {

#ifndef TC_PREFILL_STAMPS
#define TC_PREFILL_STAMPS 0  // 1: the measurement build; every prefill wave records its tile phases
#endif
constexpr int kHeadDim = 128;
// Row groups of 32 query rows per wave: each K/V fragment read from LDS
// feeds that many MFMAs.
#ifndef TC_PREFILL_GROUPS
#define TC_PREFILL_GROUPS 1
#endif
constexpr int kGroups = TC_PREFILL_GROUPS;
constexpr int kRows = 4 * 32 * kGroups;  // query rows per work-group (4 waves)
constexpr int kKeys = 64;          // keys per tile
constexpr int kRowBytes = 2 * kHeadDim;  // a K or V row in LDS (unpadded)

// TILE_CAUSAL: the tile's mask is exactly the end-aligned causal rule
// (key <= n - q_len + token), so its elements are tested arithmetically.
enum : int { TILE_SKIP = 0, TILE_FULL = 1, TILE_MIXED = 2, TILE_CAUSAL = 3 };

// Waves per SIMD the register allocation targets: 2 leaves 256 registers a
// lane and matches the two 68 KB work-groups the LDS of a CU holds.
#ifndef TC_PREFILL_WAVES
#define TC_PREFILL_WAVES 2
#endif

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

struct PrefillArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint8_t* mask;      // null, or [mb, L, n] booleans, keys contiguous (batch stride 0 broadcasts)
  const uint8_t* tiles;     // null, or the tile classes of `mask` [mb][nblk][pitch]
  uint16_t* out;            // [b, L, hq, d]
  int64_t sq_b, sq_h, sq_t;
  int64_t sk_b, sk_h, sk_t;
  int64_t sv_b, sv_h, sv_t;
  int64_t sm_b, sm_q;
  int64_t so_b, so_t, so_h;
  int64_t q_len, n;         // query tokens, keys (the queries sit at positions n - q_len ..)
  int64_t nblk, ntiles;     // query blocks per (batch, KV head); 64-key tiles of n
  int64_t pitch;            // tile map row length: ntiles rounded up to 8 (padding reads as SKIP)
  int64_t split_tiles;      // tiles per key split
  float* o_part;            // splits > 1: [b, splits, L, hq, d] fp32, normalized per split
  float* lse_part;          // splits > 1: [b, splits, L, hq] log2-sum-exp of the split (-inf if empty)
  int kv_heads, causal, neg, splits;
  int mask_words;           // mask rows 4-byte aligned: a tile's mask bytes load as words
  int whole;                // contiguous K/V: (n + 128) rows of each fit 31 bits (one buffer range a slab)
  int fold_cus;             // > 0: pair work items w and W-1-w on one CU (see the kernel), W <= 2 x this
  float c;                  // |scale| * log2(e)
  // Paged K/V (prefill_kernel<DT, G, true>): k and v are page pools whose head
  // slabs start at k + h * sk_h (v + h * sv_h); the row of sequence b's
  // logical key t sits tok_off[b * tok_pitch + t] bytes into the slab (the
  // same offset in K and V). pool_bytes_k / _v bound the buffer ranges from
  // the slab start, so a wrong offset reads zeros, not another allocation.
  const int32_t* tok_off;
  int64_t tok_pitch;
  int64_t pool_bytes_k, pool_bytes_v;
#if TC_PREFILL_STAMPS
  // Per wave (work-group * 4 + wave), kStampWords words: a header of 8 (shader
  // clock and realtime clock at the start, the same at the end, HW_REG_HW_ID
  // | HW_REG_XCC_ID << 32, tiles recorded), then 5 shader-clock stamps per
  // tile (its start, QK^T issued, softmax done, P.V issued, its loads landed).
  unsigned long long* stamps;
#endif
};
#if TC_PREFILL_STAMPS
constexpr int kStampTiles = 256;
constexpr int kStampWords = 8 + 5 * kStampTiles;
#endif

template <int DT> struct Mfma;
template <> struct Mfma<TC_DTYPE_F16> {
  static __device__ __forceinline__ float16v mma(const uint4& a, const uint4& b, const float16v& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0,
                                                  0, 0);
  }
};
template <> struct Mfma<TC_DTYPE_BF16> {
  static __device__ __forceinline__ float16v mma(const uint4& a, const uint4& b, const float16v& c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
};

// Two fp32 values rounded to nearest even into one word of two 16-bit
// elements (v_cvt_pk_f16_f32 / v_cvt_pk_bf16_f32), the first in the low half.
template <int DT> __device__ __forceinline__ uint32_t pack2(float x, float y);
template <> __device__ __forceinline__ uint32_t pack2<TC_DTYPE_F16>(float x, float y) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 v = {static_cast<_Float16>(x), static_cast<_Float16>(y)};
  return __builtin_bit_cast(uint32_t, v);
}
template <> __device__ __forceinline__ uint32_t pack2<TC_DTYPE_BF16>(float x, float y) {
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  const b2 v = {static_cast<__bf16>(x), static_cast<__bf16>(y)};
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0,
                                           static_cast<int32_t>(bytes < 0 ? 0 : (bytes > 0x7fffffff ? 0x7fffffff : bytes)),
                                           0x00020000);
}

// Paged: the offset of a key past n (as an unsigned offset, 2^31: past every
// buffer range, so the row reads zeros).
constexpr int32_t kNoRow = INT32_MIN;

// x combined with its value in lane l ^ 32 (v_permlane32_swap leaves both
// halves' values in its two results).
__device__ __forceinline__ float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The running maximum moves only when a tile's maximum exceeds it by more
// than this (log2 units), so p = exp2(s*c - m) <= 2^kLazy.
constexpr float kLazy = 8.f;

// (1, 1) as two 16-bit elements: dot2(p, kOnes) is the sum of a packed pair.
template <int DT> constexpr uint32_t kOnes = 0;
template <> constexpr uint32_t kOnes<TC_DTYPE_F16> = 0x3C003C00u;
template <> constexpr uint32_t kOnes<TC_DTYPE_BF16> = 0x3F803F80u;

// Key offset (within a 32-key half) of accumulator v of a lane in half `hi`.
__device__ __forceinline__ int acc_key(int v, int hi) { return 8 * (v >> 2) + 4 * hi + (v & 3); }

template <int DT, int G, bool PAGED>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(TC_PREFILL_WAVES, TC_PREFILL_WAVES))) void prefill_kernel(
    const PrefillArgs a) {
  constexpr int kTokens = kRows / G;   // query tokens per work-group
  // Tile buffers: K and V rows of 256 B, unpadded (a 16-byte load into LDS
  // writes 64 lanes x 16 B in one run); chunk x of row r sits in slot
  // x ^ sw(r), sw(r) = 4 (r % 4) + (r / 4) % 4, which spreads the K reads
  // (16 rows, one chunk) and the transposing V reads (8 rows, 4 chunks)
  // over all banks.
  __shared__ __attribute__((aligned(1024))) uint16_t s_k0[kKeys * kHeadDim];
  __shared__ __attribute__((aligned(1024))) uint16_t s_k1[kKeys * kHeadDim];
  __shared__ __attribute__((aligned(1024))) uint16_t s_v0[kKeys * kHeadDim];
  __shared__ __attribute__((aligned(1024))) uint16_t s_v1[kKeys * kHeadDim];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hi = lane >> 5;            // which 16 keys of each 32-key half this lane holds
  const int r32 = lane & 31;           // the lane's query row within each 32-row group
#if TC_PREFILL_STAMPS
  unsigned long long* stw = a.stamps ? a.stamps + (static_cast<int64_t>(blockIdx.x) * 4 + wave) * kStampWords : nullptr;
  int st_tile = 0;
  auto stamp = [&](int k) {
    if (stw && st_tile < kStampTiles) {
      const unsigned long long now = __builtin_amdgcn_s_memtime();
      if (lane == 0) stw[8 + 5 * st_tile + k] = now;
    }
  };
  if (stw && lane == 0) {
    stw[0] = __builtin_amdgcn_s_memtime();
    stw[1] = __builtin_amdgcn_s_memrealtime();
    unsigned hw, xcc;
    __asm__ volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
    __asm__ volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    stw[4] = hw | (static_cast<unsigned long long>(xcc) << 32);
  }
#else
  auto stamp = [](int) {};
#endif

  // Work item (KV head fastest, then key split, query block, batch):
  // consecutive work-groups go to different XCDs round-robin, so with
  // 8 | kv_heads each XCD's L2 streams one head's K/V.
  // With C CUs and a grid of C < W <= 2C work-groups (two fit a CU), the
  // dispatcher puts work-groups i and i + C on the same CU (measured on this
  // part). When the work grows along the items (causal rows see more keys),
  // fold_cus = C hands work-group i >= C item W-1-(i-C), so each CU runs item
  // i next to item W-1-i and the CUs finish together. Only the speed depends
  // on that placement.
  int64_t wid = blockIdx.x;
  if (a.fold_cus > 0 && wid >= a.fold_cus) wid = static_cast<int64_t>(gridDim.x) - 1 - (wid - a.fold_cus);
  const int h = static_cast<int>(wid % a.kv_heads);
  int64_t rest = wid / a.kv_heads;
  const int split = static_cast<int>(rest % a.splits);
  rest /= a.splits;
  int64_t blk = rest % a.nblk;
  const int b = static_cast<int>(rest / a.nblk);
  if (a.causal) blk = a.nblk - 1 - blk;  // longest rows first
  // Key and query positions and tile indices fit 32 bits (the host keeps n
  // below 2^30), so the loop's bookkeeping is 32-bit scalar arithmetic.
  const int32_t n32 = static_cast<int32_t>(a.n), q_len32 = static_cast<int32_t>(a.q_len);
  const int32_t tok0 = static_cast<int32_t>(blk) * kTokens;
  const int32_t past = n32 - q_len32;
  const int64_t bm = a.sm_b ? b : 0;

  // The wave's kGroups row groups of 32 rows: row = (token, head of the group).
  int32_t tok[kGroups];
  int hq[kGroups];
  bool row_ok[kGroups];
  const uint8_t* mrow[kGroups];
  uint4 qb[kGroups][8];  // Q^T as the MFMA B operand: dims 16c + 8*hi .. +8 of the lane's row
#pragma unroll
  for (int rg = 0; rg < kGroups; ++rg) {
    const int row = (wave * kGroups + rg) * 32 + r32;
    tok[rg] = tok0 + row / G;
    hq[rg] = h * G + row % G;
    row_ok[rg] = tok[rg] < q_len32;
    mrow[rg] = a.mask ? a.mask + bm * a.sm_b + (row_ok[rg] ? tok[rg] : 0) * a.sm_q : nullptr;
    const uint16_t* qp = a.q + b * a.sq_b + hq[rg] * a.sq_h + (row_ok[rg] ? tok[rg] : 0) * a.sq_t + 8 * hi;
    const uint32_t flip = a.neg ? 0x80008000u : 0u;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      uint4 x = row_ok[rg] ? *reinterpret_cast<const uint4*>(qp + 16 * c) : make_uint4(0u, 0u, 0u, 0u);
      x.x ^= flip; x.y ^= flip; x.z ^= flip; x.w ^= flip;
      qb[rg][c] = x;
    }
  }

  const char* kslab = reinterpret_cast<const char*>(a.k + (PAGED ? 0 : b * a.sk_b) + h * a.sk_h);
  const char* vslab = reinterpret_cast<const char*>(a.v + (PAGED ? 0 : b * a.sv_b) + h * a.sv_h);
  const int64_t row_k = a.sk_t * 2, row_v = a.sv_t * 2;
  // Buffer ranges from this head's slab on: paged, over the pools (and the
  // offsets of a tile's 64 keys, one per lane, kNoRow past n); contiguous
  // with `whole`, over the n rows (the rows past n read zeros).
  const __amdgpu_buffer_rsrc_t prk =
      rsrc(kslab, PAGED ? a.pool_bytes_k - h * a.sk_h * 2 : (a.whole ? static_cast<int64_t>(n32) * row_k : 0));
  const __amdgpu_buffer_rsrc_t prv =
      rsrc(vslab, PAGED ? a.pool_bytes_v - h * a.sv_h * 2 : (a.whole ? static_cast<int64_t>(n32) * row_v : 0));
  const int32_t* toff = PAGED ? a.tok_off + b * a.tok_pitch : nullptr;
  auto tile_rows = [&](int32_t tile) -> int32_t {
    const int32_t key = tile * kKeys + lane;
    return key < n32 ? toff[key] : kNoRow;
  };
  // Paged: when a tile's 64 keys are consecutive rows of one page (key k at
  // offset first + k * row), the offset of key 0, else -1 (also for a tile
  // that runs past n). Wave-uniform.
  auto contiguous_from = [&](int32_t idx) -> int32_t {
    const int32_t first = __builtin_amdgcn_readfirstlane(idx);
    const bool apart = static_cast<uint32_t>(idx) != static_cast<uint32_t>(first) + lane * static_cast<uint32_t>(row_k);
    return (first >= 0 && __builtin_amdgcn_ballot_w64(apart) == 0) ? first : -1;
  };
  // Load c of the eight a thread issues per tile (c < 4: K, else V), straight
  // into LDS: rows R = 16 wave + 4 (c % 4) + lane / 16, the lane filling slot
  // lane % 16 of its row with chunk (lane % 16) ^ sw(R) = (lane % 16) ^
  // (4 (lane / 16) + c % 4). Paged: a row's offset is first + key * row for a
  // contiguous tile (first >= 0), else taken from the lane of idx that holds it.
  // Contiguous: the slab's range with the tile's first row in the load's
  // scalar offset (first >= 0, `whole`), else a range over the tile's rows.
  const int dma_r = lane >> 4;
  auto dma_part = [&](uint16_t* dk, uint16_t* dv, int32_t tile, int32_t idx, int32_t first, int c) {
    const int i = c & 3;
    const int R = 16 * wave + 4 * i + dma_r;
    const int x = (lane & 15) ^ (4 * dma_r + i);
    __attribute__((address_space(3))) void* dst =
        (__attribute__((address_space(3))) void*)(reinterpret_cast<char*>(c < 4 ? dk : dv) + (16 * wave + 4 * i) * kRowBytes);
    if constexpr (PAGED) {
      if (first >= 0) {
        const int32_t row = static_cast<int32_t>(row_k);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(c < 4 ? prk : prv, dst, 16, R * row + 16 * x, first, 0, 0);
      } else {
        const int32_t off = __builtin_amdgcn_ds_bpermute(4 * R, idx) + 16 * x;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(c < 4 ? prk : prv, dst, 16, off, 0, 0, 0);
      }
    } else if (first >= 0) {
      const int32_t row = static_cast<int32_t>(c < 4 ? row_k : row_v);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(c < 4 ? prk : prv, dst, 16, R * row + 16 * x, tile * kKeys * row, 0, 0);
    } else {
      const int32_t key0 = tile * kKeys;
      const int32_t rows = n32 - key0 < kKeys ? n32 - key0 : kKeys;
      if (c < 4)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc(kslab + key0 * row_k, rows * row_k), dst, 16,
                                                 static_cast<int32_t>(R * row_k + 16 * x), 0, 0, 0);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc(vslab + key0 * row_v, rows * row_v), dst, 16,
                                                 static_cast<int32_t>(R * row_v + 16 * x), 0, 0, 0);
    }
  };
  // The eight loads of a tile. The test for a one-page tile (paged) or a
  // slab in one range (contiguous) is taken once for the burst (a test per
  // load left the compiler branching and waiting between the loads).
  auto dma_tile = [&](uint16_t* dk, uint16_t* dv, int32_t tile, int32_t idx, int32_t first) {
    if (!PAGED) first = a.whole ? 0 : -1;
    if (first >= 0) {
#pragma unroll
      for (int c = 0; c < 8; ++c) dma_part(dk, dv, tile, idx, first, c);
    } else {
#pragma unroll
      for (int c = 0; c < 8; ++c) dma_part(dk, dv, tile, idx, -1, c);
    }
  };
  const uint8_t* tcls = a.tiles ? a.tiles + (bm * a.nblk + blk) * a.pitch : nullptr;

  // Tiles this work-group may need: its split's share of all n keys, cut at
  // its last query's position when causal.
  const int32_t last_tok = min(tok0 + kTokens, q_len32) - 1;
  const int32_t key_end = a.causal ? min(n32, past + last_tok + 1) : n32;
  const int32_t split_tiles = static_cast<int32_t>(a.split_tiles);
  const int32_t t_begin = split * split_tiles;
  const int32_t nt = min((key_end + kKeys - 1) / kKeys, t_begin + split_tiles);
  // The tile map row, eight one-byte classes a word, repacked to two bits a
  // class (tile 8w + j of word w at bits 2j): the 64 words from t_begin on sit
  // one per lane and are read back with v_readlane (no memory access in the
  // loop); farther words are loaded. One register instead of two.
  const int32_t wbase = t_begin >> 3;
  auto map_load = [&](int32_t w) -> uint32_t {
    const uint64_t x = reinterpret_cast<const uint64_t*>(tcls)[w];
    uint32_t r = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) r |= static_cast<uint32_t>((x >> (8 * j)) & 3u) << (2 * j);
    return r;
  };
  const uint32_t map_pk = tcls && (wbase + lane) * 8 < a.pitch ? map_load(wbase + lane) : 0u;
  auto map_bits = [&](int32_t w) -> uint32_t {
    const int32_t i = w - wbase;
    if (i < 64) return __builtin_amdgcn_readlane(map_pk, i);
    return map_load(w);
  };
  auto tile_class = [&](int32_t t) -> int {
    if (tcls) return static_cast<int>((map_bits(t >> 3) >> (2 * (t & 7))) & 3u);
    if (a.mask) return TILE_MIXED;
    const int32_t key0 = t * kKeys;
    if (key0 + kKeys > n32) return TILE_MIXED;
    if (a.causal && key0 + kKeys - 1 > past + tok0) return TILE_MIXED;
    return TILE_FULL;
  };
  // First active tile at or after t (nt if none). With a map, eight classes
  // are tested per word (rows are 8-aligned and padded with SKIP).
  auto next_active = [&](int32_t t) -> int32_t {
    if (!tcls) {
      while (t < nt && tile_class(t) == TILE_SKIP) ++t;
      return t;
    }
    while (t < nt) {
      const uint32_t w = map_bits(t >> 3) >> (2 * (t & 7));
      if (w) return min(nt, t + (__builtin_ctz(w) >> 1));
      t = (t & ~7) + 8;
    }
    return nt;
  };

  float m[kGroups], l[kGroups];
  float16v o[kGroups][4];
#pragma unroll
  for (int rg = 0; rg < kGroups; ++rg) {
    m[rg] = neg_inf();
    l[rg] = 0.f;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int v = 0; v < 16; ++v) o[rg][dt][v] = 0.f;
  }

  // Byte offsets of the lane's K reads (chunk 2c + hi of row 32 kt + r32, kt
  // adding 8 KB) and transposing V reads (rows 16p + 8rr + 4hi + j, chunk
  // 4dt + 2(g&1) + q/2, byte 8(q&1) for lane 4j + q of 16-lane group g; p
  // adding 4 KB).
  int kaddr[8], vaddr[2][4];
  {
    const int swk = ((r32 & 3) << 2) | ((r32 >> 2) & 3);
#pragma unroll
    for (int c = 0; c < 8; ++c) kaddr[c] = r32 * kRowBytes + 16 * ((2 * c + hi) ^ swk);
    const int j = (lane & 15) >> 2, q = lane & 3, e = 2 * ((lane >> 4) & 1) + (q >> 1);
#pragma unroll
    for (int rr = 0; rr < 2; ++rr)
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
        vaddr[rr][dt] = (8 * rr + 4 * hi + j) * kRowBytes + 16 * ((4 * dt + e) ^ ((j << 2) | (2 * rr + hi))) + 8 * (q & 1);
  }

  // Active tiles t (in LDS), tn (loading) and the class of each, found one
  // iteration ahead so the tile map's reads are off the critical path.
  int32_t t = next_active(t_begin);
  int cls_t = t < nt ? tile_class(t) : TILE_SKIP;
  if (t < nt) {
    int32_t rows_t = kNoRow, first_t = -1;
    if constexpr (PAGED) {
      rows_t = tile_rows(t);
      first_t = contiguous_from(rows_t);
    }
    dma_tile(s_k0, s_v0, t, rows_t, first_t);
  }
  int32_t tn = t < nt ? next_active(t + 1) : nt;
  int cls_n = tn < nt ? tile_class(tn) : TILE_SKIP;
  // Paged: the row offsets of the tile loaded next, fetched one tile ahead.
  int32_t rows_n = kNoRow;
  if constexpr (PAGED) rows_n = tn < nt ? tile_rows(tn) : kNoRow;
  __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  // One tile from (lk, lv) while the next one loads into (dk, dv).
  auto body = [&](const uint16_t* lk, const uint16_t* lv, uint16_t* dk, uint16_t* dv) {
    stamp(0);
    const bool more = tn < nt;
    const int32_t rows_tn = rows_n;  // paged: the row offsets of tile tn, whose rows load at this tile's start
    int32_t first_tn = -1;
    if constexpr (PAGED) first_tn = more ? contiguous_from(rows_tn) : -1;
    const int32_t tnn = more ? next_active(tn + 1) : nt;
    const int cls_nn = tnn < nt ? tile_class(tnn) : TILE_SKIP;
    if constexpr (PAGED) rows_n = tnn < nt ? tile_rows(tnn) : kNoRow;
    const int cls = cls_t;

    // The next tile's eight loads per thread go out first, in one burst: spread
    // between the MFMAs below they stall the MFMA issue.
    if (more) {
      dma_tile(dk, dv, tn, rows_tn, first_tn);
    }
    // S^T of the tile for every row group: each K fragment read from LDS
    // feeds kGroups MFMAs; the two 32-key halves are independent chains.
    // The K fragments are read four chunks ahead of their MFMAs; the
    // scheduling barriers keep the compiler from pulling the reads back next
    // to their use (it otherwise waits out each read's latency).
    float16v s[kGroups][2];
#pragma unroll
    for (int rg = 0; rg < kGroups; ++rg)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int v = 0; v < 16; ++v) s[rg][kt][v] = 0.f;
    {
      auto kfrag = [&](int c, int kt) {
        return *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(lk) + kaddr[c] + 32 * kRowBytes * kt);
      };
      uint4 kf[4][2];
#pragma unroll
      for (int c = 0; c < 4; ++c) { kf[c][0] = kfrag(c, 0); kf[c][1] = kfrag(c, 1); }
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint4 k0 = kf[c & 3][0], k1 = kf[c & 3][1];
        if (c + 4 < 8) { kf[c & 3][0] = kfrag(c + 4, 0); kf[c & 3][1] = kfrag(c + 4, 1); }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int rg = 0; rg < kGroups; ++rg) {
          s[rg][0] = Mfma<DT>::mma(k0, qb[rg][c], s[rg][0]);
          s[rg][1] = Mfma<DT>::mma(k1, qb[rg][c], s[rg][1]);
        }
      }
    }

    stamp(1);
    uint4 pb[kGroups][2][2];
#pragma unroll
    for (int rg = 0; rg < kGroups; ++rg) {
      // Visible keys of this lane's row (bit 16*kt + v), all of them on a FULL tile.
      uint32_t vis = 0xffffffffu;
      float mx = neg_inf();
      if (cls != TILE_FULL) {
        const int32_t key0 = t * kKeys;
        int32_t lim = n32 - key0;
        if (a.causal || cls == TILE_CAUSAL) lim = min(lim, past + tok[rg] + 1 - key0);
        lim = max(-1, min(lim, kKeys));
        vis = 0;
        if (cls == TILE_MIXED && mrow[rg]) {
          // The row's 32 mask bytes of the tile, keys 32 kt + 8 q + 4 hi + j,
          // as one batch of loads (one wait, no branch per key): eight aligned
          // words (word q of half kt at byte 32 kt + 8 q + 4 hi) when the
          // rows are 4-byte aligned and the tile lies inside the row, else
          // 32 bytes, keys at or past lim loading the last visible key's byte
          // (key 0 when none is) so that every read stays inside the row.
          // The key < lim test hides what lies past lim.
          const uint8_t* mt = mrow[rg] + key0;
          uint32_t mw[8];
          if (a.mask_words && key0 + kKeys <= n32) {
#pragma unroll
            for (int q = 0; q < 8; ++q) mw[q] = reinterpret_cast<const uint32_t*>(mt)[2 * q + hi];
          } else {
            const int last = lim > 0 ? lim - 1 : 0;
#pragma unroll
            for (int q = 0; q < 8; ++q) {
              mw[q] = 0;
#pragma unroll
              for (int j = 0; j < 4; ++j)
                mw[q] |= static_cast<uint32_t>(mt[min(32 * (q >> 2) + 8 * (q & 3) + 4 * hi + j, last)]) << (8 * j);
            }
          }
#pragma unroll
          for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const int key = 32 * kt + acc_key(v, hi);
              const uint32_t byte = (mw[4 * kt + (v >> 2)] >> (8 * (v & 3))) & 0xffu;
              vis |= (key < lim && byte != 0) ? (1u << (16 * kt + v)) : 0u;
            }
        } else {
#pragma unroll
          for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int v = 0; v < 16; ++v) vis |= 32 * kt + acc_key(v, hi) < lim ? (1u << (16 * kt + v)) : 0u;
        }
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int v = 0; v < 16; ++v) mx = fmaxf(mx, (vis >> (16 * kt + v)) & 1u ? s[rg][kt][v] : neg_inf());
      } else {
        // Four independent max chains (fmax is exact in any order).
        float m4[4] = {s[rg][0][0], s[rg][0][1], s[rg][0][2], s[rg][0][3]};
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int v = kt ? 0 : 4; v < 16; ++v) m4[v & 3] = fmaxf(m4[v & 3], s[rg][kt][v]);
        mx = fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3]));
      }

      // Running maximum, moved only when the tile's maximum exceeds it by
      // more than 2^kLazy: p = exp2(s*c - m) then stays below 2^kLazy (exact
      // in fp16/bf16 range) and the accumulators are rescaled rarely.
      mx = pair_max(mx);
      const float tmax = mx == neg_inf() ? neg_inf() : mx * a.c;
      const bool move = tmax > m[rg] + kLazy;
      const float mn = move ? tmax : m[rg];
      const float alpha = move ? __builtin_amdgcn_exp2f(m[rg] - mn) : 1.f;
      m[rg] = mn;
      const float ms = (mn == neg_inf()) ? 0.f : mn;
      if (__builtin_amdgcn_ballot_w64(move)) {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
          for (int v = 0; v < 16; ++v) o[rg][dt][v] *= alpha;
        l[rg] *= alpha;
      }

      // P^T operand of half kt, chunk c2: accumulators 8*c2 .. 8*c2+7 are keys
      // 16*c2 + {4hi..4hi+3, 8+4hi..8+4hi+3} of the half, the order in which
      // V^T is read. All 32 exponentials come first, in one block with no
      // branch between them (a per-pair mask test would cut the block in 16
      // and leave each exp waiting on its fma); the mask then clears the
      // hidden keys in one branch. The row sum takes the rounded P, as the
      // MFMA does, in two chains (one per 32-key half).
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int v = 0; v < 16; ++v) s[rg][kt][v] = __builtin_amdgcn_exp2f(fmaf(s[rg][kt][v], a.c, -ms));
      if (cls != TILE_FULL) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int v = 0; v < 16; ++v) s[rg][kt][v] = (vis >> (16 * kt + v)) & 1u ? s[rg][kt][v] : 0.f;
      }
      float lh[2] = {0.f, 0.f};
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int c2 = 0; c2 < 2; ++c2) {
          uint32_t w[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int v0 = 8 * c2 + 2 * j;
            w[j] = pack2<DT>(s[rg][kt][v0], s[rg][kt][v0 + 1]);
            lh[kt] = Elem<DT>::dot2(w[j], kOnes<DT>, lh[kt]);
          }
          pb[rg][kt][c2] = make_uint4(w[0], w[1], w[2], w[3]);
        }
      l[rg] += lh[0] + lh[1];
    }

    stamp(2);
    // O^T += V^T . P^T: each V^T fragment read from LDS feeds kGroups MFMAs.
    // The four fragments of a 16-key step are read two steps ahead.
    {
      typedef short vs4 __attribute__((ext_vector_type(4)));
      auto vfrag = [&](int p, int dt) {
        const char* vb = reinterpret_cast<const char*>(lv) + 16 * kRowBytes * p;
        const vs4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) vs4*)(vb + vaddr[0][dt]));
        const vs4 up = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) vs4*)(vb + vaddr[1][dt]));
        const uint2 l2 = __builtin_bit_cast(uint2, lo), u2 = __builtin_bit_cast(uint2, up);
        return make_uint4(l2.x, l2.y, u2.x, u2.y);
      };
      uint4 vf[3][4];
#pragma unroll
      for (int p0 = 0; p0 < 2; ++p0)
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) vf[p0][dt] = vfrag(p0, dt);
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        if (p + 2 < 4) {
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) vf[(p + 2) % 3][dt] = vfrag(p + 2, dt);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
          for (int rg = 0; rg < kGroups; ++rg)
            o[rg][dt] = Mfma<DT>::mma(vf[p % 3][dt], pb[rg][p >> 1][p & 1], o[rg][dt]);
      }
    }

    stamp(3);
    // This thread's loads of tile tn have landed in LDS; then everyone's.
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    stamp(4);
#if TC_PREFILL_STAMPS
    ++st_tile;
#endif
    __syncthreads();
    t = tn;
    cls_t = cls_n;
    tn = tnn;
    cls_n = cls_nn;
  };
  while (t < nt) {
    body(s_k0, s_v0, s_k1, s_v1);
    if (t >= nt) break;
    body(s_k1, s_v1, s_k0, s_v0);
  }

#if TC_PREFILL_STAMPS
  if (stw && lane == 0) {
    stw[2] = __builtin_amdgcn_s_memtime();
    stw[3] = __builtin_amdgcn_s_memrealtime();
    stw[5] = static_cast<unsigned long long>(min(st_tile, kStampTiles));
  }
#endif
  // Normalize and write the lane's outputs: dims 32*dt + 8*j + 4*hi + 0..3 of each row.
#pragma unroll
  for (int rg = 0; rg < kGroups; ++rg) {
    const float lt = pair_sum(l[rg]);
    if (!row_ok[rg]) continue;
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    if (a.splits == 1) {
      uint16_t* op = a.out + b * a.so_b + tok[rg] * a.so_t + hq[rg] * a.so_h + 4 * hi;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t w0 = pack2<DT>(o[rg][dt][4 * j] * inv, o[rg][dt][4 * j + 1] * inv);
          const uint32_t w1 = pack2<DT>(o[rg][dt][4 * j + 2] * inv, o[rg][dt][4 * j + 3] * inv);
          *reinterpret_cast<uint2*>(op + 32 * dt + 8 * j) = make_uint2(w0, w1);
        }
    } else {
      // Partial of this key split, merged by prefill_combine_kernel.
      const int64_t prow =
          ((static_cast<int64_t>(b) * a.splits + split) * a.q_len + tok[rg]) * (a.kv_heads * G) + hq[rg];
      float* op = a.o_part + prow * kHeadDim + 4 * hi;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          *reinterpret_cast<float4*>(op + 32 * dt + 8 * j) = make_float4(
              o[rg][dt][4 * j] * inv, o[rg][dt][4 * j + 1] * inv, o[rg][dt][4 * j + 2] * inv,
              o[rg][dt][4 * j + 3] * inv);
      if (hi == 0) a.lse_part[prow] = lt > 0.f ? m[rg] + __log2f(lt) : neg_inf();
    }
  }
}

// out[b, tok, hq, :] = sum_s 2^(lse_s - M) o_s / sum_s 2^(lse_s - M) over the key
// splits (M = max_s lse_s); zeros when no split saw a key. 8 rows per
// 256-thread work-group, 4 dims per thread.
template <int DT>
__global__ __launch_bounds__(256) void prefill_combine_kernel(const float* o_part, const float* lse_part,
                                                              int splits, int64_t q_len, int hq_total,
                                                              uint16_t* out, int64_t so_b, int64_t so_t,
                                                              int64_t so_h) {
  const int64_t rows = q_len * hq_total;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 8 + (threadIdx.x >> 5);
  const int b = blockIdx.y;
  if (row >= rows) return;
  const int d0 = 4 * (threadIdx.x & 31);
  const float* lp = lse_part + static_cast<int64_t>(b) * splits * rows + row;
  const float* opp = o_part + (static_cast<int64_t>(b) * splits * rows + row) * kHeadDim + d0;
  // Every split's log-sum-exp and partial in one batch of loads (split s past
  // the count reads the last split again and weighs nothing), then the merge
  // in split order.
  constexpr int kMax = 16;
  float ls[kMax];
  float4 x[kMax];
#pragma unroll
  for (int s = 0; s < kMax; ++s) {
    const int si = s < splits ? s : splits - 1;
    ls[s] = lp[si * rows];
    x[s] = *reinterpret_cast<const float4*>(opp + si * rows * kHeadDim);
  }
  float mx = neg_inf();
#pragma unroll
  for (int s = 0; s < kMax; ++s) mx = s < splits ? fmaxf(mx, ls[s]) : mx;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  float wsum = 0.f;
  if (mx != neg_inf()) {
#pragma unroll
    for (int s = 0; s < kMax; ++s) {
      if (s < splits) {
        const float w = __builtin_amdgcn_exp2f(ls[s] - mx);
        acc.x += w * x[s].x; acc.y += w * x[s].y; acc.z += w * x[s].z; acc.w += w * x[s].w;
        wsum += w;
      }
    }
  }
  const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
  const int64_t tok = row / hq_total;
  const int hq = static_cast<int>(row % hq_total);
  uint16_t* op = out + b * so_b + tok * so_t + hq * so_h + d0;
  *reinterpret_cast<uint2*>(op) = make_uint2(pack2<DT>(acc.x * inv, acc.y * inv), pack2<DT>(acc.z * inv, acc.w * inv));
}

// One wave per (64-key tile, query block, mask batch): lane = key in the tile.
__global__ __launch_bounds__(64) void mask_tiles_kernel(const uint8_t* mask, int64_t sm_b, int64_t sm_q,
                                                       int64_t sm_k, int64_t q_len, int64_t n, int tokens,
                                                       int64_t nblk, int64_t pitch, uint8_t* tiles) {
  const int lane = threadIdx.x;
  const int64_t t = blockIdx.x, blk = blockIdx.y, bm = blockIdx.z;
  const int64_t key = t * kKeys + lane;
  const int64_t tok0 = blk * tokens;
  const int64_t tok_end = min(tok0 + tokens, q_len);
  const int64_t past = n - q_len;
  bool any = false, all = key < n, causal = true;
  if (key < n) {
    const uint8_t* p = mask + bm * sm_b + key * sm_k;
    for (int64_t tok = tok0; tok < tok_end; ++tok) {
      const bool x = p[tok * sm_q] != 0;
      any |= x;
      all &= x;
      causal &= x == (key <= past + tok);
    }
  }
  const uint64_t any_w = __builtin_amdgcn_ballot_w64(any);
  const uint64_t all_w = __builtin_amdgcn_ballot_w64(all);
  const uint64_t causal_w = __builtin_amdgcn_ballot_w64(causal);
  if (lane == 0) {
    const int cls = any_w == 0                  ? TILE_SKIP
                    : all_w == ~uint64_t(0)     ? TILE_FULL
                    : causal_w == ~uint64_t(0)  ? TILE_CAUSAL
                                                : TILE_MIXED;
    tiles[(bm * nblk + blk) * pitch + t] = static_cast<uint8_t>(cls);
  }
}

#if TC_PREFILL_STAMPS
unsigned long long* g_prefill_stamps = nullptr;  // the buffer prefill launches record into (null: none)
#endif

template <int DT, bool PAGED>
void launch_attention(const PrefillArgs& a_in, int group, dim3 grid, hipStream_t stream) {
  PrefillArgs a = a_in;
#if TC_PREFILL_STAMPS
  a.stamps = g_prefill_stamps;
#endif
  switch (group) {
    case 1: hipLaunchKernelGGL((prefill_kernel<DT, 1, PAGED>), grid, dim3(256), 0, stream, a); break;
    case 2: hipLaunchKernelGGL((prefill_kernel<DT, 2, PAGED>), grid, dim3(256), 0, stream, a); break;
    case 4: hipLaunchKernelGGL((prefill_kernel<DT, 4, PAGED>), grid, dim3(256), 0, stream, a); break;
    default: hipLaunchKernelGGL((prefill_kernel<DT, 8, PAGED>), grid, dim3(256), 0, stream, a); break;
  }
}

template <int DT>
hipError_t launch_dt(const PrefillArgs& a, int group, int batch, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(a.nblk * a.kv_heads * batch * a.splits));
  if (a.tok_off)
    launch_attention<DT, true>(a, group, grid, stream);
  else
    launch_attention<DT, false>(a, group, grid, stream);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.splits == 1) return e;
  const int hq_total = a.kv_heads * group;
  const dim3 cgrid(static_cast<unsigned>((a.q_len * hq_total + 7) / 8), static_cast<unsigned>(batch));
  hipLaunchKernelGGL((prefill_combine_kernel<DT>), cgrid, dim3(256), 0, stream, a.o_part, a.lse_part, a.splits,
                     a.q_len, hq_total, a.out, a.so_b, a.so_t, a.so_h);
  return hipGetLastError();
}

int check3(const char* what, const int64_t* st) {
  if (!st) return fail(TC_ERR_INVALID_ARGUMENT, "%s strides are null", what);
  for (int i = 0; i < 3; ++i) {
    if (st[i] < 0) return fail(TC_ERR_INVALID_ARGUMENT, "%s stride %d negative", what, i);
    if (st[i] % 8) return fail(TC_ERR_ALIGNMENT, "%s stride %d (%lld) not a multiple of 8", what, i, (long long)st[i]);
  }
  return TC_OK;
}

int check_group(int q_heads, int kv_heads, int* group) {
  if (kv_heads < 1 || kv_heads > 65535 || q_heads < 1)
    return fail(TC_ERR_INVALID_ARGUMENT, "q_heads %d, kv_heads %d", q_heads, kv_heads);
  if (q_heads % kv_heads)
    return fail(TC_ERR_INVALID_ARGUMENT, "q_heads %d not a multiple of kv_heads %d", q_heads, kv_heads);
  *group = q_heads / kv_heads;
  if (*group != 1 && *group != 2 && *group != 4 && *group != 8)
    return fail(TC_ERR_UNSUPPORTED, "group %d unsupported (1, 2, 4 or 8)", *group);
  return TC_OK;
}

int check_mask_strides(const int64_t* st) {
  if (!st) return fail(TC_ERR_INVALID_ARGUMENT, "mask strides are null");
  if (st[0] < 0 || st[1] < 0 || st[2] < 0) return fail(TC_ERR_INVALID_ARGUMENT, "mask strides must be non-negative");
  if (st[2] != 1) return fail(TC_ERR_UNSUPPORTED, "mask keys must be contiguous (key stride %lld)", (long long)st[2]);
  return TC_OK;
}

// Tile map geometry: query blocks of 128/g tokens, 64-key tiles.
int64_t map_pitch(int64_t ntiles) { return (ntiles + 7) & ~int64_t(7); }

void tile_geometry(int64_t q_len, int64_t n, int group, int64_t* nblk, int64_t* ntiles) {
  const int64_t tokens = kRows / group;
  *nblk = (q_len + tokens - 1) / tokens;
  *ntiles = (n + kKeys - 1) / kKeys;
}

constexpr int kMaxPrefillSplits = 16;
static_assert(kMaxPrefillSplits <= 16, "prefill_combine_kernel loads at most 16 splits");
constexpr int kMinSplitTiles = 4;    // keys per split: at least 256

// Key splits of a call: 1 when the query blocks alone give every CU two
// work-groups or the chunk is at least half its keys, else as many as still fit the CUs' two work-group slots in one
// round (each split at least kMinSplitTiles tiles, at most kMaxPrefillSplits):
// a work-group more than the slots would run in a second round and double the
// call. requested > 0 overrides the choice. Trailing empty splits are dropped:
// the result times its tiles covers n.
int plan_splits(int batch, int64_t q_len, int64_t n, int group, int kv_heads, int requested, int64_t* split_tiles,
                int* splits_out) {
  int64_t nblk, ntiles;
  tile_geometry(q_len, n, group, &nblk, &ntiles);
  int64_t s = 1;
  if (requested > 0) {
    s = requested;
  } else {
    int cus = 0;
    const int rc = current_device_cus(&cus);
    if (rc != TC_OK) return rc;
    // Work-groups resident per CU: one per wave slot of a SIMD (4 waves each).
    const int64_t wgs = nblk * kv_heads * batch, slots = TC_PREFILL_WAVES * static_cast<int64_t>(cus);
    if (wgs < slots) s = slots / wgs;
    s = std::min<int64_t>(s, std::max<int64_t>(1, ntiles / kMinSplitTiles));
    // A chunk that is half of its keys or more (a prompt) runs unsplit: its
    // work-groups hold few tiles, and the combine costs more than the split
    // saves (1024-token prompt: 28 us unsplit, 43 us in two splits).
    if (2 * q_len >= n) s = 1;
  }
  s = std::max<int64_t>(1, std::min<int64_t>({s, kMaxPrefillSplits, std::max<int64_t>(1, ntiles)}));
  const int64_t st = std::max<int64_t>(1, (ntiles + s - 1) / s);
  *split_tiles = st;
  *splits_out = static_cast<int>(std::max<int64_t>(1, (ntiles + st - 1) / st));
  return TC_OK;
}

size_t workspace_bytes(int batch, int64_t q_len, int q_heads, int splits) {
  if (splits <= 1) return 0;
  return static_cast<size_t>(batch) * splits * q_len * q_heads * (kHeadDim + 1) * sizeof(float);
}

}  // namespace
}  // namespace tc

using namespace tc;

extern "C" int tc_prefill_num_splits(int batch, int64_t q_len, int64_t n_tokens, int q_heads, int kv_heads) {
  clear_error();
  int group = 0, rc;
  if (batch < 1 || q_len < 0 || n_tokens < q_len) return -fail(TC_ERR_INVALID_ARGUMENT, "batch %d, q_len %lld, n %lld", batch, (long long)q_len, (long long)n_tokens);
  if ((rc = check_group(q_heads, kv_heads, &group)) != TC_OK) return -rc;
  int64_t st;
  int splits;
  if ((rc = plan_splits(batch, q_len, n_tokens, group, kv_heads, 0, &st, &splits)) != TC_OK) return -rc;
  return splits;
}

extern "C" size_t tc_prefill_workspace_bytes(int batch, int64_t q_len, int q_heads, int num_splits) {
  if (batch < 1 || q_len < 0 || q_heads < 1) return 0;
  return workspace_bytes(batch, q_len, q_heads, num_splits);
}

extern "C" size_t tc_prefill_tiles_bytes(int64_t q_len, int64_t n_tokens, int mask_batch, int q_heads,
                                         int kv_heads) {
  int group = 0;
  if (q_len < 0 || n_tokens < q_len || mask_batch < 1 || check_group(q_heads, kv_heads, &group) != TC_OK) return 0;
  int64_t nblk, ntiles;
  tile_geometry(q_len, n_tokens, group, &nblk, &ntiles);
  return static_cast<size_t>(mask_batch * nblk * map_pitch(ntiles));
}

extern "C" int tc_prefill_mask_tiles(const uint8_t* mask_dev, const int64_t mask_strides[3], int mask_batch,
                                     int64_t q_len, int64_t n_tokens, int q_heads, int kv_heads, uint8_t* tiles_dev,
                                     size_t tiles_bytes, void* stream) {
  clear_error();
  int group = 0, rc;
  if ((rc = check_group(q_heads, kv_heads, &group)) != TC_OK) return rc;
  if (mask_batch < 1 || mask_batch > 65535) return fail(TC_ERR_INVALID_ARGUMENT, "mask_batch %d", mask_batch);
  if (q_len < 0 || n_tokens < q_len)
    return fail(TC_ERR_INVALID_ARGUMENT, "q_len %lld must be in [0, n_tokens %lld]", (long long)q_len,
                (long long)n_tokens);
  if ((rc = check_mask_strides(mask_strides)) != TC_OK) return rc;
  if (mask_batch > 1 && mask_strides[0] == 0)
    return fail(TC_ERR_INVALID_ARGUMENT, "mask_batch %d with a broadcast (stride 0) mask batch", mask_batch);
  int64_t nblk, ntiles;
  tile_geometry(q_len, n_tokens, group, &nblk, &ntiles);
  const int64_t pitch = map_pitch(ntiles);
  const size_t need = static_cast<size_t>(mask_batch * nblk * pitch);
  if (need == 0) return TC_OK;
  if (!mask_dev || !tiles_dev) return fail(TC_ERR_INVALID_ARGUMENT, "null mask or tile map pointer");
  if (tiles_bytes < need)
    return fail(TC_ERR_WORKSPACE, "tile map holds %zu bytes, needs %zu", tiles_bytes, need);
  if (ntiles > 0x7fffffff || nblk > 65535)
    return fail(TC_ERR_UNSUPPORTED, "mask of %lld x %lld exceeds the tile grid", (long long)q_len,
                (long long)n_tokens);
  if (reinterpret_cast<uintptr_t>(tiles_dev) & 7u) return fail(TC_ERR_ALIGNMENT, "tile map must be 8-byte aligned");
  // The padding tiles (keys past n) classify as SKIP, so whole rows are written.
  const dim3 grid(static_cast<unsigned>(pitch), static_cast<unsigned>(nblk), static_cast<unsigned>(mask_batch));
  hipLaunchKernelGGL(mask_tiles_kernel, grid, dim3(64), 0, static_cast<hipStream_t>(stream), mask_dev,
                     mask_strides[0], mask_strides[1], mask_strides[2], q_len, n_tokens, kRows / group, nblk, pitch,
                     tiles_dev);
  return hip_status(hipGetLastError(), "mask tile launch");
}

namespace tc {
namespace {

// The page pools of a paged prefill call.
struct PagedPools {
  const int32_t* tok_off;  // [batch, tok_pitch] byte offsets of each logical key's row in its head slab
  int64_t tok_pitch;
  int64_t pool_bytes;      // bytes of one pool (K and V pools share the shape)
};

int prefill_impl(const void* q_dev, const int64_t q_strides[3], const void* k_dev, const int64_t k_strides[3],
                 const void* v_dev, const int64_t v_strides[3], const uint8_t* mask_dev,
                 const int64_t mask_strides[3], const uint8_t* mask_tiles_dev, size_t mask_tiles_bytes, int causal,
                 int64_t q_len, int64_t n_tokens, int batch, int q_heads, int kv_heads, int head_dim, int dtype,
                 float scale, int num_splits, void* workspace_dev, size_t workspace_bytes_in, void* out_dev,
                 const int64_t out_strides[3], void* stream, const PagedPools* pools) {
  int group = 0, rc;
  if (batch < 1 || batch > 65535) return fail(TC_ERR_INVALID_ARGUMENT, "batch %d", batch);
  if ((rc = check_group(q_heads, kv_heads, &group)) != TC_OK) return rc;
  if (head_dim != kHeadDim) return fail(TC_ERR_UNSUPPORTED, "head_dim %d unsupported (kernels are built for 128)", head_dim);
  if (dtype != TC_DTYPE_F16 && dtype != TC_DTYPE_BF16) return fail(TC_ERR_UNSUPPORTED, "dtype %d unsupported", dtype);
  if (q_len < 0 || n_tokens < q_len)
    return fail(TC_ERR_INVALID_ARGUMENT, "q_len %lld must be in [0, n_tokens %lld]", (long long)q_len,
                (long long)n_tokens);
  if (q_len == 0) return TC_OK;
  // Key positions and tile indices are 32-bit in the kernel.
  if (n_tokens >= (int64_t(1) << 30))
    return fail(TC_ERR_UNSUPPORTED, "n_tokens %lld: the prefill kernels take fewer than 2^30 keys", (long long)n_tokens);
  if (!q_dev || !k_dev || !v_dev || !out_dev) return fail(TC_ERR_INVALID_ARGUMENT, "null tensor pointer");
  if (!aligned16(q_dev) || !aligned16(k_dev) || !aligned16(v_dev) || !aligned16(out_dev))
    return fail(TC_ERR_ALIGNMENT, "q/k/v/out base pointers must be 16-byte aligned");
  if ((rc = check3("q", q_strides)) != TC_OK) return rc;
  if ((rc = check3("k", k_strides)) != TC_OK) return rc;
  if ((rc = check3("v", v_strides)) != TC_OK) return rc;
  if ((rc = check3("out", out_strides)) != TC_OK) return rc;
  // A 64-key tile is addressed with 32-bit buffer offsets: 64 rows of at most 2^24 elements.
  constexpr int64_t kMaxTokenStride = int64_t(1) << 24;
  if (k_strides[2] < head_dim || v_strides[2] < head_dim || k_strides[2] >= kMaxTokenStride ||
      v_strides[2] >= kMaxTokenStride)
    return fail(TC_ERR_INVALID_ARGUMENT, "k/v token strides outside [%d, 2^24)", head_dim);
  if (!std::isfinite(scale)) return fail(TC_ERR_INVALID_ARGUMENT, "scale is not finite");
  int64_t nblk, ntiles;
  tile_geometry(q_len, n_tokens, group, &nblk, &ntiles);
  if (nblk * kv_heads * batch * kMaxPrefillSplits > 0x7fffffff) return fail(TC_ERR_UNSUPPORTED, "grid too large");
  if (mask_dev) {
    if (causal) return fail(TC_ERR_INVALID_ARGUMENT, "pass either a mask or causal, not both");
    if ((rc = check_mask_strides(mask_strides)) != TC_OK) return rc;
    if (mask_tiles_dev) {
      const size_t need = static_cast<size_t>((mask_strides[0] ? batch : 1) * nblk * map_pitch(ntiles));
      if (reinterpret_cast<uintptr_t>(mask_tiles_dev) & 7u)
        return fail(TC_ERR_ALIGNMENT, "tile map must be 8-byte aligned");
      if (mask_tiles_bytes < need)
        return fail(TC_ERR_WORKSPACE, "tile map holds %zu bytes, this call reads %zu", mask_tiles_bytes, need);
    }
  } else if (mask_tiles_dev) {
    return fail(TC_ERR_INVALID_ARGUMENT, "a tile map without its mask");
  }

  int64_t split_tiles;
  int splits;
  if ((rc = plan_splits(batch, q_len, n_tokens, group, kv_heads, num_splits, &split_tiles, &splits)) != TC_OK)
    return rc;
  const size_t need = workspace_bytes(batch, q_len, q_heads, splits);
  if (need > 0 && (!workspace_dev || workspace_bytes_in < need))
    return fail(TC_ERR_WORKSPACE, "%d key splits need %zu workspace bytes, got %zu", splits, need,
                workspace_dev ? workspace_bytes_in : size_t(0));
  if (need > 0 && (reinterpret_cast<uintptr_t>(workspace_dev) & 15u))
    return fail(TC_ERR_ALIGNMENT, "workspace must be 16-byte aligned");

  PrefillArgs a;
  a.split_tiles = split_tiles;
  a.splits = splits;
  a.o_part = static_cast<float*>(workspace_dev);
  a.lse_part = splits > 1 ? a.o_part + static_cast<size_t>(batch) * splits * q_len * q_heads * kHeadDim : nullptr;
  a.q = static_cast<const uint16_t*>(q_dev);
  a.k = static_cast<const uint16_t*>(k_dev);
  a.v = static_cast<const uint16_t*>(v_dev);
  a.mask = mask_dev;
  a.tiles = mask_dev ? mask_tiles_dev : nullptr;
  a.out = static_cast<uint16_t*>(out_dev);
  a.sq_b = q_strides[0]; a.sq_h = q_strides[1]; a.sq_t = q_strides[2];
  a.sk_b = k_strides[0]; a.sk_h = k_strides[1]; a.sk_t = k_strides[2];
  a.sv_b = v_strides[0]; a.sv_h = v_strides[1]; a.sv_t = v_strides[2];
  a.sm_b = mask_dev ? mask_strides[0] : 0;
  a.sm_q = mask_dev ? mask_strides[1] : 0;
  a.mask_words = mask_dev && reinterpret_cast<uintptr_t>(mask_dev) % 4 == 0 && a.sm_b % 4 == 0 && a.sm_q % 4 == 0;
  a.whole = !pools && (n_tokens + 2 * kKeys) * 2 * std::max(k_strides[2], v_strides[2]) < (int64_t(1) << 31);
  a.so_b = out_strides[0]; a.so_t = out_strides[1]; a.so_h = out_strides[2];
  a.q_len = q_len;
  a.n = n_tokens;
  a.nblk = nblk;
  a.ntiles = ntiles;
  a.pitch = map_pitch(ntiles);
  a.kv_heads = kv_heads;
  a.causal = causal ? 1 : 0;
  a.fold_cus = 0;
  if (splits == 1 && (causal || mask_dev)) {
    // One round of two work-groups per CU with rows that see more keys further down.
    int cus = 0;
    if ((rc = current_device_cus(&cus)) != TC_OK) return rc;
    const int64_t wgs = nblk * kv_heads * batch, slots = TC_PREFILL_WAVES * static_cast<int64_t>(cus);
    if (wgs > cus && wgs <= slots) a.fold_cus = cus;
  }
  a.neg = scale < 0.f ? 1 : 0;
  a.c = static_cast<float>(std::fabs(static_cast<double>(scale)) * 1.4426950408889634);
  a.tok_off = pools ? pools->tok_off : nullptr;
  a.tok_pitch = pools ? pools->tok_pitch : 0;
  a.pool_bytes_k = a.pool_bytes_v = pools ? pools->pool_bytes : 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const hipError_t e = dtype == TC_DTYPE_F16 ? launch_dt<TC_DTYPE_F16>(a, group, batch, s)
                                             : launch_dt<TC_DTYPE_BF16>(a, group, batch, s);
  return hip_status(e, "prefill launch");
}

}  // namespace
}  // namespace tc

extern "C" int tc_prefill_attention(const void* q_dev, const int64_t q_strides[3], const void* k_dev,
                                    const int64_t k_strides[3], const void* v_dev, const int64_t v_strides[3],
                                    const uint8_t* mask_dev, const int64_t mask_strides[3],
                                    const uint8_t* mask_tiles_dev, size_t mask_tiles_bytes, int causal,
                                    int64_t q_len, int64_t n_tokens, int batch, int q_heads, int kv_heads,
                                    int head_dim, int dtype, float scale, int num_splits, void* workspace_dev,
                                    size_t workspace_bytes_in, void* out_dev, const int64_t out_strides[3],
                                    void* stream) {
  clear_error();
  return prefill_impl(q_dev, q_strides, k_dev, k_strides, v_dev, v_strides, mask_dev, mask_strides, mask_tiles_dev,
                      mask_tiles_bytes, causal, q_len, n_tokens, batch, q_heads, kv_heads, head_dim, dtype, scale,
                      num_splits, workspace_dev, workspace_bytes_in, out_dev, out_strides, stream, nullptr);
}

extern "C" int tc_prefill_paged_attention(const void* q_dev, const int64_t q_strides[3], const void* k_pool_dev,
                                          const void* v_pool_dev, const int64_t pool_strides[3], int num_pages,
                                          const int32_t* tok_off_dev, int64_t tok_pitch, const uint8_t* mask_dev,
                                          const int64_t mask_strides[3], const uint8_t* mask_tiles_dev,
                                          size_t mask_tiles_bytes, int causal, int64_t q_len, int64_t n_tokens,
                                          int batch, int q_heads, int kv_heads, int head_dim, int dtype, float scale,
                                          int num_splits, void* workspace_dev, size_t workspace_bytes_in,
                                          void* out_dev, const int64_t out_strides[3], void* stream) {
  clear_error();
  if (!pool_strides) return fail(TC_ERR_INVALID_ARGUMENT, "null pool strides");
  if (num_pages < 1) return fail(TC_ERR_INVALID_ARGUMENT, "pool of %d pages", num_pages);
  if (q_len > 0 && (!tok_off_dev || tok_pitch < n_tokens))
    return fail(TC_ERR_INVALID_ARGUMENT, "token offsets: null or a row of %lld for %lld keys", (long long)tok_pitch,
                (long long)n_tokens);
  if (reinterpret_cast<uintptr_t>(tok_off_dev) & 3u) return fail(TC_ERR_ALIGNMENT, "token offsets not 4-byte aligned");
  // Rows are found by 32-bit byte offsets from a head's slab.
  const int64_t pool_bytes = static_cast<int64_t>(num_pages) * pool_strides[0] * 2;
  if (pool_strides[0] < 1 || pool_bytes >= (int64_t(1) << 31) ||
      static_cast<int64_t>(kv_heads - 1) * pool_strides[1] * 2 >= pool_bytes)
    return fail(TC_ERR_UNSUPPORTED, "pool of %lld bytes (page stride %lld): paged prefill needs a pool under 2 GiB",
                (long long)pool_bytes, (long long)pool_strides[0]);
  const PagedPools pools{tok_off_dev, tok_pitch, pool_bytes};
  return prefill_impl(q_dev, q_strides, k_pool_dev, pool_strides, v_pool_dev, pool_strides, mask_dev, mask_strides,
                      mask_tiles_dev, mask_tiles_bytes, causal, q_len, n_tokens, batch, q_heads, kv_heads, head_dim,
                      dtype, scale, num_splits, workspace_dev, workspace_bytes_in, out_dev, out_strides, stream,
                      &pools);
}

#if TC_PREFILL_STAMPS
// Measurement build only (libthreadcut_stamps.so): the device buffer that the
// prefill kernels launched from now on record their per-wave, per-tile phase
// stamps into (kStampWords words per wave, see PrefillArgs::stamps), or null.
extern "C" void tc_prefill_set_stamps(void* stamps_dev) {
  tc::g_prefill_stamps = static_cast<unsigned long long*>(stamps_dev);
}
#endif
