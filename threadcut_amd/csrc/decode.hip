// Split-KV GQA flash-decode for gfx950: a partial online-softmax kernel over
// (split, kv head, sequence) work-groups on the matrix cores, and a separate
// log-sum-exp combine.
//
// Reference semantics: threadcut/flash_decode.py:21-54 (`_partial`: fp32
// softmax, scale applied after q.k, -inf guards, out = acc / l,
// lse = m + log l) and :57-69 (decode_attention: splits = cdiv(n, split),
// merge with softmax(lse) weights, cast to q.dtype).
//
// Per wave and 16-token tile, with n = lane % 16 (query head: a column of
// every 16x16 MFMA block; columns n >= G hold zeros) and g = lane / 16:
//   S^T[token][head] = K[token][:] . Q[head][:]   four v_mfma_f32_16x16x32
//     (k = 32 dims each). A = K rows: lane l loads token l % 16, bytes
//     [64 i + 16 g, +16) of its row for block i, so each load instruction
//     reads 16 rows x 64 contiguous bytes; B = Q with the same dims, held in
//     registers for the whole kernel. Lane l receives S^T[4g + r][n], r < 4.
//   softmax per head in fp32, log2 domain, the tile maximum across the four
//     lane groups by two permlane swaps; the running maximum moves only when
//     a tile's exceeds it by 2^8 (p is then at most 2^8), so the accumulators
//     are rescaled rarely.
//   O^T[dim][head] += V^T[dim][token] . P^T[token][head]   eight
//     v_mfma_f32_16x16x16 (k = 16 tokens), each twice: with P rounded to the
//     element type and with the rounding residue, so the weights carry about
//     16 (bf16) or 22 (fp16) significant bits. P^T leaves the S^T registers as
//     the B operand without moving between lanes (lane l holds tokens
//     4g..4g+3 of head n in both layouts). V is loaded as 4 tokens x 8 dims
//     per lane and stored row-major to the wave's own LDS region (16-byte
//     stores, rows padded to 288 bytes); the A operand V^T comes back through
//     the transposing ds_read_b64_tr_b16, so V is never transposed in
//     registers.
// The matrix core sums over a wave's tokens, so a wave's accumulator is
// complete; the four waves of a work-group are merged through LDS and the
// work-group writes one (o, lse) partial per query head.

#include <math.h>

#include <algorithm>
#include <mutex>

#include "tc_common.hpp"

namespace tc {
namespace {

// Tuning knobs (measured on MI355X; override with -D for sweeps).
#ifndef TC_DECODE_WAVES
#define TC_DECODE_WAVES 4   // waves per partial work-group
#endif
#ifndef TC_DECODE_AUX
#define TC_DECODE_AUX 2     // cache-policy bits of the K/V buffer loads (2: non-temporal stream)
#endif
#ifndef TC_DECODE_INTERLEAVE
#define TC_DECODE_INTERLEAVE 1  // tc_decode_attention deals tiles round-robin over the splits
#endif
#ifndef TC_DECODE_RAGGED_WGS_PER_CU
#define TC_DECODE_RAGGED_WGS_PER_CU 8  // the same with per-sequence lengths: finer splits balance them
#endif
#ifndef TC_DECODE_WGS_PER_CU
#define TC_DECODE_WGS_PER_CU 1  // partial work-groups per compute unit the split heuristic aims at
#endif
#ifndef TC_DECODE_WPE
#define TC_DECODE_WPE 1  // amdgpu_waves_per_eu floor of the partial kernel (2 caps a wave at 256 registers)
#endif
#ifndef TC_DECODE_WPE_PAGED
#define TC_DECODE_WPE_PAGED 2  // the same for the paged instantiations
#endif
#ifndef TC_DECODE_STAMPS
#define TC_DECODE_STAMPS 0  // 1: the measurement build; every partial wave records a timeline
#endif

constexpr int kHeadDim = 128;
constexpr int64_t kMaxTokens = int64_t(1) << 29;  // token positions stay 32-bit in the kernel
constexpr int kWaves = TC_DECODE_WAVES;
constexpr int kThreads = 64 * kWaves;
// Short caches (at most TC_DECODE_SHORT_TOKENS tokens, one length for the
// batch): partial work-groups of two waves over the same splits. A wave then
// has two tiles where it had one, and the merge of two waves costs less than
// that of four (36 layers, Qwen3-4B heads, call us: 512 tokens 5.76 against
// 5.87, 1024 5.89 against 6.02, 1536 6.05 against 6.25, 2048 6.50 against
// 6.84; at 3072 and 4096 tokens two waves are slower).
constexpr int kShortWaves = 2;
constexpr int kWaveIter = 16;                        // tokens per wave iteration
constexpr int kSplitGranule = kWaves * kWaveIter > 64 ? kWaves * kWaveIter : 64;  // split length granule
static_assert(kSplitGranule % (kShortWaves * kWaveIter) == 0, "short plans split at the same granule");
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

struct PartialArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  float* o_part;       // [B, H, S, G, D]
  float* lse_part;     // [B, H, S, G]
  const int32_t* lens; // [B] or null
  int64_t n;
  int64_t sq_b, sq_h, sq_g;
  int64_t sk_b, sk_h, sk_t;
  int64_t sv_b, sv_h, sv_t;
  int heads, group, splits, split_tokens;
  int interleave;      // 0: split s owns tokens [s*T, (s+1)*T); 1: 16-token tiles dealt round-robin
  int longest_first;   // per-sequence lengths, batch <= 64: work-group row z serves the z-th longest sequence
  float scale_log2;    // softmax scale * log2(e)
  // Append (k_new != null): the cache holds n - 1 tokens and the new token's
  // K/V rows [B, H, D] are attended from k_new/v_new and written to row n - 1
  // of the cache (k_w/v_w) by wave 0 of split 0; no other wave reads that row.
  const uint16_t* k_new;
  const uint16_t* v_new;
  int64_t skn_b, skn_h, svn_b, svn_h;
  uint16_t* k_w;
  uint16_t* v_w;
  // Paged cache (decode_partial_kernel<DT, true, *>): k and v are page pools
  // [pages, H, P, D] with element strides (sk_b, sk_h, sk_t) = (page, head,
  // token). Sequence b's keys are the tiles tile_tab[b * max_tiles + i],
  // i < tiles[b], each {page, first slot, rows, 0}: rows (<= 16) consecutive
  // slots of one page. Entries outside the pool or the page count as empty.
  const int32_t* tile_tab;
  const int32_t* tiles;
  int64_t max_tiles;
  int32_t pages, page_tokens;
  // Paged append with device lengths (tok_off != null): sequence b holds
  // lens[b] tokens before this step; tile entries carry their first logical
  // position in the 4th word, and a tile's rows are those below lens[b]
  // (tiles reserved ahead read nothing). The new token goes to logical
  // position lens[b], whose row sits tok_off[b * tok_pitch + lens[b]] bytes
  // into the head slab of the pools.
  const int32_t* tok_off;
  int64_t tok_pitch;
#if TC_DECODE_STAMPS
  // Per wave ((b * heads + h) * splits + split) * waves + wave, 8 words:
  // realtime-clock stamps (100 MHz) at the kernel's start, after the first
  // tile's step, at the loop's end, after the merge barrier and after the
  // partial stores are issued, then HW_REG_HW_ID and HW_REG_XCC_ID.
  unsigned long long* stamps;
#endif
};

struct CombineArgs {
  const float* o_part;
  const float* lse_part;
  uint16_t* out;
  int64_t so_b, so_h, so_g;
  int heads, group, splits;
};

// Reductions over the four 16-lane rows of a wave (every lane gets the result).
// v_permlane16_swap(x, x) leaves rows (x0, x0, x2, x2) and (x1, x1, x3, x3) in its two
// results, so their sum is x0 + x1 (x2 + x3) in every lane; permlane32 pairs the halves.
__device__ __forceinline__ float pair16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float pair16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float rows_sum(float x) { return pair32_sum(pair16_sum(x)); }
__device__ __forceinline__ float rows_max(float x) { return pair32_max(pair16_max(x)); }

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// A wave-uniform read of memory that no kernel writes while this one runs:
// through the constant address space it becomes a scalar load.
__device__ __forceinline__ int32_t const_load(const int32_t* p) {
  return *reinterpret_cast<const __attribute__((address_space(4))) int32_t*>(reinterpret_cast<uintptr_t>(p));
}

// Buffer resource over `bytes` bytes at p; loads past the end return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, int32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, 0x00020000);
}

__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, int32_t off) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, TC_DECODE_AUX);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// K/V of one 16-token tile of a wave (lane l = 16 g + n): k[i] = token n,
// dims 32 i + 8 g .. +8 (the A operand of QK block i); v[j] = token 4 g + j,
// dims 8 n .. +8. Rows at or past `end` read as zero (their scores are
// masked), so no index clamping is needed.
struct Tile {
  uint4 k[4];
  uint4 v[4];
  int32_t rows;  // paged cache: the tile's key rows (the rest read as zero)
};

__device__ __forceinline__ void load_tile(Tile& t, const char* kslab, const char* vslab, int32_t row_k,
                                          int32_t row_v, int32_t t0, int32_t end, const int32_t* koff,
                                          const int32_t* voff) {
  // The clamp is wave-uniform, but i32 min/max select v_med3 (a VGPR);
  // readfirstlane keeps the buffer resource in SGPRs (no waterfall loop).
  const int32_t rows = __builtin_amdgcn_readfirstlane(min(max(end - t0, 0), 16));
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kslab + static_cast<int64_t>(t0) * row_k, rows * row_k);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(vslab + static_cast<int64_t>(t0) * row_v, rows * row_v);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    t.k[j] = bload16(rk, koff[j]);
    t.v[j] = bload16(rv, voff[j]);
  }
}

// Paged cache: rows (<= 16) key rows from slot `slot` of page `page`. The
// buffer range spans exactly those rows, so the rest of the tile reads as
// zero; an entry outside the pool or past the page's end loads nothing.
__device__ __forceinline__ void load_paged_tile(Tile& t, const char* kpool, const char* vpool, int32_t row_k,
                                                int32_t row_v, int64_t page_k, int64_t page_v, int32_t pages,
                                                int32_t page_tokens, int32_t page, int32_t slot, int32_t rows,
                                                const int32_t* koff, const int32_t* voff) {
  if (page < 0 || page >= pages || slot < 0 || rows < 0 || rows > 16 || slot > page_tokens - rows) {
    page = 0; slot = 0; rows = 0;
  }
  t.rows = rows;
  const __amdgpu_buffer_rsrc_t rk = make_rsrc(kpool + page * page_k + static_cast<int64_t>(slot) * row_k, rows * row_k);
  const __amdgpu_buffer_rsrc_t rv = make_rsrc(vpool + page * page_v + static_cast<int64_t>(slot) * row_v, rows * row_v);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    t.k[j] = bload16(rk, koff[j]);
    t.v[j] = bload16(rv, voff[j]);
  }
}

typedef _Float16 mfma_h4 __attribute__((ext_vector_type(4)));
typedef _Float16 mfma_h8 __attribute__((ext_vector_type(8)));
typedef __bf16 mfma_b8 __attribute__((ext_vector_type(8)));
typedef short mfma_s4 __attribute__((ext_vector_type(4)));
typedef float mfma_f4 __attribute__((ext_vector_type(4)));

template <int DT> struct DecodeMma;
template <> struct DecodeMma<TC_DTYPE_F16> {
  static __device__ __forceinline__ mfma_f4 qk(const uint4& a, const uint4& b, const mfma_f4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(mfma_h8, a), __builtin_bit_cast(mfma_h8, b), c,
                                                  0, 0, 0);
  }
  static __device__ __forceinline__ mfma_f4 pv(const uint2& a, const uint2& b, const mfma_f4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(mfma_h4, a), __builtin_bit_cast(mfma_h4, b), c,
                                                 0, 0, 0);
  }
  // Two fp32 values rounded to nearest even into one word (first in the low half).
  static __device__ __forceinline__ uint32_t pack(float x, float y) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 v = {static_cast<_Float16>(x), static_cast<_Float16>(y)};
    return __builtin_bit_cast(uint32_t, v);
  }
};
template <> struct DecodeMma<TC_DTYPE_BF16> {
  static __device__ __forceinline__ mfma_f4 qk(const uint4& a, const uint4& b, const mfma_f4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(mfma_b8, a), __builtin_bit_cast(mfma_b8, b), c,
                                                   0, 0, 0);
  }
  static __device__ __forceinline__ mfma_f4 pv(const uint2& a, const uint2& b, const mfma_f4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(mfma_s4, a), __builtin_bit_cast(mfma_s4, b),
                                                     c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float x, float y) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    const b2 v = {static_cast<__bf16>(x), static_cast<__bf16>(y)};
    return __builtin_bit_cast(uint32_t, v);
  }
};

// Row-major V tile in a wave's LDS region: 16 token rows of 256 bytes, each
// padded to 288 so that the transposing reads (4 rows x 32 bytes per 16-lane
// group, 16 rows per instruction) and the 16-byte row stores fall on distinct
// banks.
constexpr int kVRowBytes = 2 * kHeadDim + 32;
constexpr int kVTileWords = 16 * kVRowBytes / 4;
typedef short lds_s4 __attribute__((ext_vector_type(4)));
constexpr float kLazyMax = 8.f;               // log2 units the running maximum may lag

// APPEND: the kernel attends (and writes) the new token of an append call
// (a.k_new != null); the other instantiation carries none of that code.
template <int DT, bool PAGED, bool APPEND, int W>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(PAGED ? TC_DECODE_WPE_PAGED : TC_DECODE_WPE))) void decode_partial_kernel(const PartialArgs a) {
  using M = DecodeMma<DT>;
  using E = Elem<DT>;
  // W waves per work-group (kWaves, or kShortWaves for short caches).
  __shared__ uint32_t s_vt[W][kVTileWords];
  // The merge's rows are padded by 16 words, so the float4 stores of the g
  // heads (one head per 16 lanes) fall on distinct banks.
  __shared__ float s_acc[W][8][kHeadDim + 16];
  __shared__ float s_m[8][W];
  __shared__ float s_l[8][W];

#if TC_DECODE_STAMPS
  const unsigned long long st_start = __builtin_amdgcn_s_memrealtime();
  unsigned long long st_first = 0, st_loop = 0, st_merge = 0;
#endif
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15;   // head column (also the token row of the K operand)
  const int g = lane >> 4;   // lane group
  // Grid (heads, splits, batch), the KV head fastest: consecutive work-groups
  // go to consecutive XCDs, so with 8 KV heads every split of head h runs on
  // XCD h and its partials stay in that XCD's L2 for the combine.
  const int h = blockIdx.x;
  const int split = blockIdx.y;
  // With per-sequence lengths the work-groups of the z-th longest sequence
  // take grid row z, so the longest sequences are dispatched first (ties by
  // index): lane j ranks sequence j by length, and the ballot finds the lane
  // of rank z.
  int b = blockIdx.z;
  int32_t len_b = 0;  // longest-first: sequence b's length, read with the others
  if (!PAGED && a.longest_first) {
    const int B = static_cast<int>(gridDim.z);
    const int32_t mine = lane < B ? a.lens[lane] : 0;
    int rank = 0;
    for (int i = 0; i < B; ++i) {
      const int32_t other = __builtin_amdgcn_readlane(mine, i);
      rank += (other > mine || (other == mine && i < lane)) ? 1 : 0;
    }
    const uint64_t hit = __builtin_amdgcn_ballot_w64(lane < B && rank == static_cast<int>(blockIdx.z));
    b = hit ? __builtin_ctzll(hit) : b;
    len_b = __builtin_amdgcn_readlane(mine, b);
  }

  // Paged: the pools' head slabs, pages added per tile; otherwise sequence b's slabs.
  const char* kslab = reinterpret_cast<const char*>(a.k + (PAGED ? 0 : b * a.sk_b) + h * a.sk_h);
  const char* vslab = reinterpret_cast<const char*>(a.v + (PAGED ? 0 : b * a.sv_b) + h * a.sv_h);
  const int32_t row_k = static_cast<int32_t>(a.sk_t) * 2, row_v = static_cast<int32_t>(a.sv_t) * 2;
  __asm__ volatile("" ::"s"(kslab), "s"(vslab));
  const int32_t nt = static_cast<int32_t>(a.n);
  const int32_t len_cap = APPEND ? nt - 1 : nt;
  // The wave's first tile and the distance between its tiles.
  int32_t tok, tok_step, wave_tokens = 0;
  if (a.interleave) {
    tok = (split * W + wave) * kWaveIter;
    tok_step = a.splits * W * kWaveIter;
  } else {
    wave_tokens = a.split_tokens / W;
    tok = split * a.split_tokens + wave * wave_tokens;
    tok_step = kWaveIter;
  }
  const int32_t* tab = PAGED ? a.tile_tab + static_cast<int64_t>(b) * a.max_tiles * 4 : nullptr;
  // Paged: lane i holds the table entry of the wave's i-th tile (tiles past
  // the 64th read theirs from memory). The entries are requested before the
  // tile count is known, bounded by the table's row, so the two reads are in
  // flight together.
  int32_t e_page = 0, e_slot = 0, e_cnt = 0, e_pos = 0;
  const int32_t ti = tok + lane * tok_step;
  if constexpr (PAGED) {
    if ((ti >> 4) < a.max_tiles) {
      const int4 e = *reinterpret_cast<const int4*>(tab + 4 * (ti >> 4));
      e_page = e.x; e_slot = e.y; e_cnt = e.z; e_pos = e.w;
    }
  }
  int32_t len = len_cap;
  int32_t last_tile = -1;  // paged append: the tile whose last row is the new token's slot
  int32_t plen = -1;  // paged append with device lengths: tokens cached before this step
  if constexpr (PAGED) {
    // Token index space of 16 per tile; a tile's own row count masks the rest.
    // The tile count and lengths are read with scalar loads (constant for the
    // kernel's lifetime).
    const int32_t ntiles = min(max(const_load(a.tiles + b), 0), static_cast<int32_t>(a.max_tiles));
    len = 16 * ntiles;
    if (a.tok_off) plen = max(const_load(a.lens + b), 0);
    else if (APPEND)
      last_tile = ntiles - 1;
  } else if (a.lens) {
    len = min(max(a.longest_first ? len_b : a.lens[b], 0), len_cap);
  }
  const int32_t end = a.interleave ? len : min(tok + wave_tokens, len);

  // K: token n of the tile, bytes [64 i + 16 g, +16) for block i.
  // V: tokens 4g + j, dims 8n .. 8n + 7.
  int32_t koff[4], voff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    koff[i] = n * row_k + 64 * i + 16 * g;
    voff[i] = (4 * g + i) * row_v + 16 * n;
  }
  // Rows each preloaded tile contributes: none past the wave's tiles; the
  // append's last tile less the new token's row (attended from k_new); with
  // device lengths, the rows below lens[b].
  int32_t e_rows = 0;
  if constexpr (PAGED) {
    if (ti < end) {
      e_rows = (ti >> 4) == last_tile ? e_cnt - 1 : e_cnt;
      if (plen >= 0) e_rows = min(e_cnt, max(plen - e_pos, 0));
    }
  }
  int32_t li = 0;  // the wave's tiles loaded so far
  auto load = [&](Tile& tl, int32_t t0) {
    if constexpr (PAGED) {
      int32_t page = 0, slot = 0, rows = 0;
      if (li < 64) {
        page = __builtin_amdgcn_readlane(e_page, li);
        slot = __builtin_amdgcn_readlane(e_slot, li);
        rows = __builtin_amdgcn_readlane(e_rows, li);
      } else if (t0 < end) {
        const int4 e = *reinterpret_cast<const int4*>(tab + 4 * (t0 >> 4));
        page = __builtin_amdgcn_readfirstlane(e.x);
        slot = __builtin_amdgcn_readfirstlane(e.y);
        int32_t r = (t0 >> 4) == last_tile ? e.z - 1 : e.z;
        if (plen >= 0) r = min(e.z, max(plen - e.w, 0));
        rows = __builtin_amdgcn_readfirstlane(r);
      }
      ++li;
      load_paged_tile(tl, kslab, vslab, row_k, row_v, a.sk_b * 2, a.sv_b * 2, a.pages, a.page_tokens, page, slot,
                      rows, koff, voff);
    } else {
      load_tile(tl, kslab, vslab, row_k, row_v, t0, end, koff, voff);
    }
  };
  Tile t[2];
  load(t[0], tok);

  // Q as the B operand: head n, dims 32 i + 8 g .. +8 (zero for n >= G).
  uint4 qb[4];
  {
    const uint16_t* qrow = a.q + b * a.sq_b + h * a.sq_h + n * a.sq_g + 8 * g;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      qb[i] = make_uint4(0u, 0u, 0u, 0u);
      if (n < a.group) qb[i] = *reinterpret_cast<const uint4*>(qrow + 32 * i);
    }
  }

  mfma_f4 acc[8];
#pragma unroll
  for (int bm = 0; bm < 8; ++bm) acc[bm] = mfma_f4{0.f, 0.f, 0.f, 0.f};
  float m = neg_inf(), l = 0.f;

  // One 16-token tile whose first token is t0 (tokens >= lim are masked).
  auto step = [&](const Tile& tl, int32_t t0, int32_t lim) {
    // S^T block: two independent chains of two MFMAs each.
    mfma_f4 s0 = M::qk(tl.k[0], qb[0], mfma_f4{0.f, 0.f, 0.f, 0.f});
    mfma_f4 s1 = M::qk(tl.k[1], qb[1], mfma_f4{0.f, 0.f, 0.f, 0.f});
    s0 = M::qk(tl.k[2], qb[2], s0);
    s1 = M::qk(tl.k[3], qb[3], s1);
    // V into LDS, row-major, while the matrix core works: lane (g, n)
    // stores tokens 4g + j, dims 8n .. 8n + 7.
    char* vrow = reinterpret_cast<char*>(s_vt[wave]);
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<uint4*>(vrow + (4 * g + j) * kVRowBytes + 16 * n) = tl.v[j];
    float x[4];
#pragma unroll
    for (int r = 0; r < 4; ++r)
      x[r] = (t0 + 4 * g + r < lim) ? (s0[r] + s1[r]) * a.scale_log2 : neg_inf();
    const float tmax = rows_max(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])));
    // Lazy running maximum: moves only when the tile's exceeds it by kLazyMax.
    const float mn = (tmax > m + kLazyMax || m == neg_inf()) ? tmax : m;
    const float ms = (mn == neg_inf()) ? 0.f : mn;
    // Rescale what was accumulated (nothing while m is still -inf: acc and l are zero).
    if (__any(mn != m && m != neg_inf())) {
      const float alpha = __builtin_amdgcn_exp2f(m - ms);  // 0 while nothing was seen
#pragma unroll
      for (int bm = 0; bm < 8; ++bm) acc[bm] *= alpha;
      l *= alpha;
    }
    m = mn;
    float p[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) p[r] = __builtin_amdgcn_exp2f(x[r] - ms);
    l += (p[0] + p[1]) + (p[2] + p[3]);
    const uint32_t h01 = M::pack(p[0], p[1]), h23 = M::pack(p[2], p[3]);
    const uint32_t r01 = M::pack(p[0] - E::lo(h01), p[1] - E::hi(h01));
    const uint32_t r23 = M::pack(p[2] - E::lo(h23), p[3] - E::hi(h23));
    const uint2 phi = make_uint2(h01, h23), plo = make_uint2(r01, r23);
#pragma unroll
    for (int bm = 0; bm < 8; ++bm) {
      // A operand V^T[16 bm + n][4g .. 4g + 3]: ds_read_b64_tr_b16 hands lane n
      // of a 16-lane group element (n % 4) of what lane 4 j + n / 4 addressed,
      // for j = 0..3; lane (g, n) addresses row 4g + n / 4, dims 16 bm + 4 (n % 4).
      const lds_s4 t4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) lds_s4*)(vrow + (4 * g + (n >> 2)) * kVRowBytes + 32 * bm + 8 * (n & 3)));
      const uint2 av = __builtin_bit_cast(uint2, t4);
      acc[bm] = M::pv(av, phi, acc[bm]);
      acc[bm] = M::pv(av, plo, acc[bm]);
    }
  };

  // Two tiles in flight: the next tile's loads are issued before the current
  // tile is consumed, and no load is issued past the wave's last tile.
  if (tok < end) {
    for (;;) {
      const int32_t tok1 = tok + tok_step, tok2 = tok1 + tok_step;
      load(t[1], tok1);
      step(t[0], tok, PAGED ? tok + t[0].rows : end);
#if TC_DECODE_STAMPS
      if (st_first == 0) st_first = __builtin_amdgcn_s_memrealtime();
#endif
      load(t[0], tok2);
      if (tok1 < end) step(t[1], tok1, PAGED ? tok1 + t[1].rows : end);
      tok = tok2;
      if (tok >= end) break;
    }
  }

  if (APPEND && split == 0 && wave == 0) {
    // The appended token as a tile whose only row is token 0 (the buffer
    // range is one row, so the other rows read zero and are masked).
    const char* kn = reinterpret_cast<const char*>(a.k_new + b * a.skn_b + h * a.skn_h);
    const char* vn = reinterpret_cast<const char*>(a.v_new + b * a.svn_b + h * a.svn_h);
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(kn, kHeadDim * 2);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vn, kHeadDim * 2);
    Tile tn;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      tn.k[j] = bload16(rk, 64 * j + 16 * g + n * kHeadDim * 2);
      tn.v[j] = bload16(rv, (4 * g + j) * kHeadDim * 2 + 16 * n);
    }
    step(tn, 0, 1);
    if (lane < 32) {
      const bool is_v = lane >= 16;
      const int chunk = 8 * (lane & 15);
      const uint16_t* src = is_v ? a.v_new + b * a.svn_b + h * a.svn_h : a.k_new + b * a.skn_b + h * a.skn_h;
      uint16_t* dst = nullptr;
      if constexpr (PAGED) {
        // The new token's slot: with device lengths, the offset table's row of
        // position lens[b] (a position past the table's rows, or an offset
        // outside the pool, writes nothing); otherwise the last row of the
        // sequence's last tile (an invalid entry, or no tile, writes nothing).
        if (plen >= 0) {
          const int32_t off = plen < a.tok_pitch ? a.tok_off[static_cast<int64_t>(b) * a.tok_pitch + plen] : -1;
          const int64_t room = static_cast<int64_t>(a.pages) * a.sk_b * 2 - h * a.sk_h * 2 - kHeadDim * 2;
          if (off >= 0 && off <= room) {
            char* base = reinterpret_cast<char*>(is_v ? a.v_w + h * a.sv_h : a.k_w + h * a.sk_h);
            dst = reinterpret_cast<uint16_t*>(base + off);
          }
        } else if (last_tile >= 0) {
          const int4 e = *reinterpret_cast<const int4*>(tab + 4 * last_tile);
          if (!(e.x < 0 || e.x >= a.pages || e.y < 0 || e.z < 1 || e.z > 16 || e.y > a.page_tokens - e.z)) {
            const int64_t slot = e.y + e.z - 1;
            dst = is_v ? a.v_w + e.x * a.sv_b + h * a.sv_h + slot * a.sv_t
                       : a.k_w + e.x * a.sk_b + h * a.sk_h + slot * a.sk_t;
          }
        }
      } else {
        dst = is_v ? a.v_w + b * a.sv_b + h * a.sv_h + len * a.sv_t : a.k_w + b * a.sk_b + h * a.sk_h + len * a.sk_t;
      }
      if (dst) *reinterpret_cast<uint4*>(dst + chunk) = *reinterpret_cast<const uint4*>(src + chunk);
    }
  }

#if TC_DECODE_STAMPS
  st_loop = __builtin_amdgcn_s_memrealtime();
  auto record = [&]() {
    if (a.stamps && lane == 0) {
      unsigned long long* o =
          a.stamps + (((static_cast<int64_t>(b) * a.heads + h) * a.splits + split) * W + wave) * 8;
      o[0] = st_start; o[1] = st_first; o[2] = st_loop; o[3] = st_merge;
      o[4] = __builtin_amdgcn_s_memrealtime();
      o[5] = __builtin_amdgcn_s_getreg((31 << 11) | (0 << 6) | 4);   // HW_REG_HW_ID
      o[6] = __builtin_amdgcn_s_getreg((15 << 11) | (0 << 6) | 20);  // HW_REG_XCC_ID
    }
  };
#endif
  // The head's sum over the four lane groups; m is already common to them.
  l = rows_sum(l);
  const int64_t part = (static_cast<int64_t>(b) * a.heads + h) * a.splits + split;
  if constexpr (W == 1) {
    // One wave: its accumulator is the split's; lane (g, n) holds dims
    // 16 bm + 4 g .. + 3 of head n.
    if (n < a.group) {
      const float inv = l == 0.f ? 0.f : __builtin_amdgcn_rcpf(l);
      float* o = a.o_part + (part * a.group + n) * kHeadDim + 4 * g;
#pragma unroll
      for (int bm = 0; bm < 8; ++bm)
        *reinterpret_cast<float4*>(o + 16 * bm) =
            make_float4(acc[bm][0] * inv, acc[bm][1] * inv, acc[bm][2] * inv, acc[bm][3] * inv);
      if (g == 0) a.lse_part[part * a.group + n] = (l == 0.f) ? neg_inf() : (m + __builtin_amdgcn_logf(l)) * kLn2;
    }
#if TC_DECODE_STAMPS
    st_merge = st_loop;
    record();
#endif
    return;
  }
  if (n < a.group) {
#pragma unroll
    for (int bm = 0; bm < 8; ++bm)
      *reinterpret_cast<float4*>(&s_acc[wave][n][16 * bm + 4 * g]) =
          make_float4(acc[bm][0], acc[bm][1], acc[bm][2], acc[bm][3]);
    if (g == 0) { s_m[n][wave] = m; s_l[n][wave] = l; }
  }
  // The split's output rows, addressed before the barrier (the address
  // arithmetic is then off the path from the barrier to the stores).
  float* const o_out = a.o_part + part * a.group * kHeadDim;
  float* const l_out = a.lse_part + part * a.group;
  __asm__ volatile("" ::"s"(o_out), "s"(l_out));
  __syncthreads();
#if TC_DECODE_STAMPS
  st_merge = __builtin_amdgcn_s_memrealtime();
#endif

  // Each thread merges two adjacent dims of one head (one pass for G <= 4).
  for (int idx = threadIdx.x; idx < a.group * (kHeadDim / 2); idx += 64 * W) {
    const int hh = idx / (kHeadDim / 2);
    const int d = 2 * (idx % (kHeadDim / 2));
    float mw[W], lw[W];
    float2 ow[W];
#pragma unroll
    for (int w = 0; w < W; ++w) {
      mw[w] = s_m[hh][w];
      lw[w] = s_l[hh][w];
      ow[w] = *reinterpret_cast<const float2*>(&s_acc[w][hh][d]);
    }
    float Mx = neg_inf();
#pragma unroll
    for (int w = 0; w < W; ++w) Mx = fmaxf(Mx, mw[w]);
    const float Ms = (Mx == neg_inf()) ? 0.f : Mx;
    float L = 0.f, O0 = 0.f, O1 = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float f = __builtin_amdgcn_exp2f(mw[w] - Ms);
      L += lw[w] * f;
      O0 += ow[w].x * f;
      O1 += ow[w].y * f;
    }
    // L >= 1 whenever a token was seen (the maximum contributes exp2(0)).
    const float inv = L == 0.f ? 0.f : __builtin_amdgcn_rcpf(L);
    *reinterpret_cast<float2*>(o_out + hh * kHeadDim + d) = make_float2(O0 * inv, O1 * inv);
    if (d == 0) l_out[hh] = (L == 0.f) ? neg_inf() : (Mx + __builtin_amdgcn_logf(L)) * kLn2;
  }
#if TC_DECODE_STAMPS
  record();
#endif
}

// x of the lane pair (l, l ^ 16) or (l, l ^ 32): the lower row's value in lo,
// the upper row's in hi, in both lanes.
template <bool ROW32>
__device__ __forceinline__ void swap_pair(float x, float& lo, float& hi) {
  const uint32_t u = __float_as_uint(x);
  const auto r = ROW32 ? __builtin_amdgcn_permlane32_swap(u, u, false, false)
                       : __builtin_amdgcn_permlane16_swap(u, u, false, false);
  lo = __uint_as_float(r[0]);
  hi = __uint_as_float(r[1]);
}

// x of lanes l and l ^ K (K = 8: DPP row rotate by 8; 16, 32: permlane swaps),
// the lower lane's value in lo, the upper lane's in hi, in both lanes.
template <int K>
__device__ __forceinline__ void lane_pair(float x, int lane, float& lo, float& hi) {
  if constexpr (K == 8) {
    const float o = __uint_as_float(__builtin_amdgcn_mov_dpp(__float_as_uint(x), 0x128, 0xf, 0xf, false));  // row_ror:8
    const bool upper = (lane & 8) != 0;
    lo = upper ? o : x;
    hi = upper ? x : o;
  } else {
    swap_pair<K == 32>(x, lo, hi);
  }
}
// One merge step of the (max, sum, weighted o) states of lanes l and l ^ K,
// lower lane first, so both lanes hold the same bits afterwards.
template <int K>
__device__ __forceinline__ void combine_merge(float& M, float& L, float4& O, int lane) {
  float m0, m1, x0, x1;
  lane_pair<K>(M, lane, m0, m1);
  const float Mx = fmaxf(m0, m1);
  const float Ms = (Mx == neg_inf()) ? 0.f : Mx;
  const float f0 = __builtin_amdgcn_exp2f((m0 - Ms) * kLog2e);
  const float f1 = __builtin_amdgcn_exp2f((m1 - Ms) * kLog2e);
  lane_pair<K>(L, lane, x0, x1); L = x0 * f0 + x1 * f1;
  lane_pair<K>(O.x, lane, x0, x1); O.x = x0 * f0 + x1 * f1;
  lane_pair<K>(O.y, lane, x0, x1); O.y = x0 * f0 + x1 * f1;
  lane_pair<K>(O.z, lane, x0, x1); O.z = x0 * f0 + x1 * f1;
  lane_pair<K>(O.w, lane, x0, x1); O.w = x0 * f0 + x1 * f1;
  M = Mx;
}

// Combine: one wave per (sequence, KV head, query head, quarter of the dims),
// grid (heads, batch, group * 4), the KV head fastest, so with 8 heads head
// h's waves run on XCD h, where the partial kernel wrote its partials. Lane
// (sg, chunk) takes dims 32 q + 4 chunk .. + 3 of splits sg, sg + 8, sg + 16,
// ...: four splits a lane per round of 32, every load of a round issued before
// the first is consumed (one memory round trip per round). Each round folds
// its splits into a running (max, sum, weighted o) with one exponential per
// split; the eight split groups are then merged across lanes (a DPP row
// rotate, permlane16 and permlane32 swaps). Spreading a head's dims over four
// waves keeps each wave's loads to 8 a round (the one-wave-per-head form
// issued 32).
template <int DT>
__global__ __launch_bounds__(64) void decode_combine_kernel(const CombineArgs a) {
  using E = Elem<DT>;
  constexpr int kPer = 4;  // splits a lane loads per round
  const int lane = threadIdx.x;
  const int chunk = lane & 7;
  const int sg = lane >> 3;
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int g = blockIdx.z >> 2;
  const int qtr = blockIdx.z & 3;
  const int G = a.group;
  const int S = a.splits;
  const int64_t bh = static_cast<int64_t>(b) * a.heads + h;
  // Buffer ranges over this (sequence, head)'s partials: loads past them read zero.
  const __amdgpu_buffer_rsrc_t ro = make_rsrc(a.o_part + bh * S * G * kHeadDim, S * G * kHeadDim * 4);
  const __amdgpu_buffer_rsrc_t rl = make_rsrc(a.lse_part + bh * S * G, S * G * 4);
  // Per-lane byte offsets (split sg of a round); the round's split r0 + 8 j
  // adds a wave-uniform offset.
  const int32_t o_split = G * kHeadDim * 4;  // bytes between splits
  const int32_t o_lane = sg * o_split + (g * kHeadDim + 32 * qtr + 4 * chunk) * 4;
  const int32_t l_lane = (sg * G + g) * 4;

  float M = neg_inf(), L = 0.f;
  float4 O = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int r0 = 0; r0 < S; r0 += 8 * kPer) {
    u32x4 ov[kPer];
    float ls[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int32_t s0 = r0 + 8 * j;
      // The buffer range check covers the scalar offset too (measured on
      // gfx950), so splits past S read zero.
      ov[j] = __builtin_amdgcn_raw_buffer_load_b128(ro, o_lane, s0 * o_split, 0);
      ls[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rl, l_lane, s0 * G * 4, 0));
    }
    // Every load of the round is in flight before the first is consumed.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < kPer; ++j)
      if (r0 + 8 * j + sg >= S) ls[j] = neg_inf();  // past the last split (the load read zero)
    float mr = ls[0];
#pragma unroll
    for (int j = 1; j < kPer; ++j) mr = fmaxf(mr, ls[j]);
    const float Mn = fmaxf(M, mr);
    const float Ms = (Mn == neg_inf()) ? 0.f : Mn;
    const float f = __builtin_amdgcn_exp2f((M - Ms) * kLog2e);  // 0 while nothing was seen
    L *= f;
    O.x *= f; O.y *= f; O.z *= f; O.w *= f;
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const float w = __builtin_amdgcn_exp2f((ls[j] - Ms) * kLog2e);
      L += w;
      O.x += w * __uint_as_float(ov[j].x);
      O.y += w * __uint_as_float(ov[j].y);
      O.z += w * __uint_as_float(ov[j].z);
      O.w += w * __uint_as_float(ov[j].w);
    }
    M = Mn;
  }
  // Merge the split groups: lanes l ^ 8, l ^ 16 and l ^ 32.
  combine_merge<8>(M, L, O, lane);
  combine_merge<16>(M, L, O, lane);
  combine_merge<32>(M, L, O, lane);
  if (sg == 0) {
    // An empty cache (no splits, or every split empty) gives zeros.
    const float inv = (M == neg_inf()) ? 0.f : 1.f / L;
    const uint32_t w0 = E::bits(O.x * inv) | (E::bits(O.y * inv) << 16);
    const uint32_t w1 = E::bits(O.z * inv) | (E::bits(O.w * inv) << 16);
    uint16_t* dst = a.out + b * a.so_b + h * a.so_h + g * a.so_g + 32 * qtr + 4 * chunk;
    *reinterpret_cast<uint2*>(dst) = make_uint2(w0, w1);
  }
}

// ---------------------------------------------------------------------------
// Host-side validation and launch.
// ---------------------------------------------------------------------------

#if TC_DECODE_STAMPS
unsigned long long* g_stamps = nullptr;  // the stamp buffer partial launches record into (null: none)
#endif

int check_strides(const char* what, const int64_t* st, int n) {
  if (!st) return fail(TC_ERR_INVALID_ARGUMENT, "%s strides are null", what);
  for (int i = 0; i < n; ++i) {
    if (st[i] < 0) return fail(TC_ERR_INVALID_ARGUMENT, "%s stride %d is negative (%lld)", what, i, (long long)st[i]);
    if (st[i] % 8 != 0)
      return fail(TC_ERR_ALIGNMENT, "%s stride %d (%lld elements) is not a multiple of 8", what, i, (long long)st[i]);
  }
  return TC_OK;
}

int check_common(int batch, int kv_heads, int group, int head_dim, int dtype) {
  if (batch < 1 || batch > 65535) return fail(TC_ERR_INVALID_ARGUMENT, "batch %d outside [1, 65535]", batch);
  if (kv_heads < 1 || kv_heads > 65535) return fail(TC_ERR_INVALID_ARGUMENT, "kv_heads %d outside [1, 65535]", kv_heads);
  if (group < 1 || group > 8) return fail(TC_ERR_UNSUPPORTED, "group (query heads per KV head) %d outside [1, 8]", group);
  if (head_dim != kHeadDim) return fail(TC_ERR_UNSUPPORTED, "head_dim %d unsupported (kernels are built for 128)", head_dim);
  if (dtype != TC_DTYPE_F16 && dtype != TC_DTYPE_BF16) return fail(TC_ERR_UNSUPPORTED, "dtype %d unsupported", dtype);
  return TC_OK;
}

inline dim3 partial_grid(const PartialArgs& a, int batch) { return dim3(a.heads, a.splits, batch); }

template <int DT, bool PAGED>
void launch_partial_paged(const PartialArgs& a, int batch, int waves, hipStream_t stream) {
  if (a.k_new) {
    hipLaunchKernelGGL((decode_partial_kernel<DT, PAGED, true, kWaves>), partial_grid(a, batch), dim3(kThreads), 0,
                       stream, a);
    return;
  }
  if constexpr (!PAGED) {
    if (waves == kShortWaves) {
      hipLaunchKernelGGL((decode_partial_kernel<DT, false, false, kShortWaves>), partial_grid(a, batch),
                         dim3(64 * kShortWaves), 0, stream, a);
      return;
    }
  }
  hipLaunchKernelGGL((decode_partial_kernel<DT, PAGED, false, kWaves>), partial_grid(a, batch), dim3(kThreads), 0,
                     stream, a);
}

template <int DT>
hipError_t launch_partial_dt(const PartialArgs& a, int batch, int waves, hipStream_t stream) {
  if (a.tile_tab)
    launch_partial_paged<DT, true>(a, batch, waves, stream);
  else
    launch_partial_paged<DT, false>(a, batch, waves, stream);
  return hipGetLastError();
}

// Waves per partial work-group: two for a short cache with one length for the
// batch, read by the plain call with its tiles dealt round-robin; else four.
inline int partial_waves(int64_t n_tokens, bool lens, bool paged, bool append, int interleave) {
  return (interleave && !lens && !paged && !append && n_tokens <= TC_DECODE_SHORT_TOKENS) ? kShortWaves : kWaves;
}

// Split plan of a call: S splits of T tokens each (S * T >= n, T a multiple of
// the granule). With split_tokens > 0 the caller fixes T. Otherwise S is
// chosen so that B * Hkv * S work-groups are TC_DECODE_WGS_PER_CU per compute
// unit (every work-group then streams the same share of the cache when its
// tiles are dealt round-robin), but never more splits than a head has
// wave-tiles and never more than TC_MAX_SPLITS. Ragged batches (per-sequence
// lengths) aim at TC_DECODE_RAGGED_WGS_PER_CU per unit: short sequences leave
// their work-groups light, and many small work-groups let the dispatcher
// balance the rest. The plan does not depend on the work-group shape: a short
// cache read by two-wave work-groups keeps the four-wave plan's splits (its
// waves then take two tiles each where four-wave ones took one).
int split_plan(int batch, int kv_heads, int64_t max_tokens, int split_tokens, int ragged, int* S_out, int* T_out) {
  if (batch < 1 || kv_heads < 1 || max_tokens < 0)
    return fail(TC_ERR_INVALID_ARGUMENT, "split query with batch %d, kv_heads %d, max_tokens %lld", batch, kv_heads,
                (long long)max_tokens);
  // Shortest split that keeps the split count within TC_MAX_SPLITS.
  const int64_t floor_t = ceil_div(ceil_div(max_tokens, TC_MAX_SPLITS), kSplitGranule) * kSplitGranule;
  int64_t t, S;
  if (split_tokens > 0) {
    t = max(ceil_div(split_tokens, kSplitGranule) * kSplitGranule, floor_t);
    S = ceil_div(max_tokens, t);
  } else {
    int cus = 0;
    const int rc = current_device_cus(&cus);
    if (rc != TC_OK) return rc;
    const int64_t target = static_cast<int64_t>(ragged ? TC_DECODE_RAGGED_WGS_PER_CU : TC_DECODE_WGS_PER_CU) * cus;
    const int64_t per_head = static_cast<int64_t>(batch) * kv_heads;
    const int64_t max_s = std::max<int64_t>(1, std::min<int64_t>(ceil_div(ceil_div(max_tokens, kWaveIter), kWaves),
                                                        TC_MAX_SPLITS));
    S = std::max<int64_t>(1, std::min<int64_t>((target + per_head / 2) / per_head, max_s));
    t = max(ceil_div(ceil_div(max_tokens, S), kSplitGranule) * kSplitGranule, floor_t);
    if (max_tokens == 0) S = 0;
  }
  t = max(t, static_cast<int64_t>(kSplitGranule));
  if (t > (1 << 30)) return fail(TC_ERR_INVALID_ARGUMENT, "split length %lld too large", (long long)t);
  *S_out = static_cast<int>(S);
  *T_out = static_cast<int>(t);
  return TC_OK;
}

}  // namespace
}  // namespace tc

using namespace tc;

extern "C" {

int tc_decode_split_tokens(int batch, int kv_heads, int64_t max_tokens, int split_tokens, int ragged) {
  clear_error();
  int S = 0, t = 0;
  const int rc = split_plan(batch, kv_heads, max_tokens, split_tokens, ragged, &S, &t);
  return rc == TC_OK ? t : -rc;
}

int tc_decode_num_splits(int batch, int kv_heads, int64_t max_tokens, int split_tokens, int ragged) {
  clear_error();
  int S = 0, t = 0;
  const int rc = split_plan(batch, kv_heads, max_tokens, split_tokens, ragged, &S, &t);
  return rc == TC_OK ? S : -rc;
}

size_t tc_decode_workspace_bytes(int batch, int kv_heads, int group, int head_dim, int num_splits) {
  if (batch < 1 || kv_heads < 1 || group < 1 || head_dim < 1 || num_splits < 0) return 0;
  const size_t parts = static_cast<size_t>(batch) * kv_heads * num_splits * group;
  return parts * head_dim * sizeof(float) + parts * sizeof(float);
}

}  // extern "C"

namespace tc {
namespace {

// The new token of an append-and-attend call: K/V rows [B, H, D] and the
// writable cache they go to.
struct Append {
  const void* k_new;
  const int64_t* kn_strides;  // (batch, head)
  const void* v_new;
  const int64_t* vn_strides;
  void* k_cache;
  void* v_cache;
};

// A paged cache: the tile table of every sequence and the pool's shape.
struct Paged {
  const int32_t* tile_tab;  // [B, max_tiles, 4]
  const int32_t* tiles;     // [B]
  int64_t max_tiles;
  int pages, page_tokens;
  const int32_t* tok_off = nullptr;  // device-length append: [B, tok_pitch] row byte offsets
  int64_t tok_pitch = 0;
};

int partial_impl(const void* q_dev, const int64_t q_strides[3], const void* k_dev, const int64_t k_strides[3],
                 const void* v_dev, const int64_t v_strides[3], const int32_t* lens_dev, int64_t n_tokens, int batch,
                 int kv_heads, int group, int head_dim, int dtype, float scale, int split_tokens, int num_splits,
                 float* o_part_dev, float* lse_part_dev, int interleave, const Append* app, void* stream,
                 const Paged* paged = nullptr) {
  int rc = check_common(batch, kv_heads, group, head_dim, dtype);
  if (rc != TC_OK) return rc;
  if (n_tokens == 0 && num_splits == 0) return TC_OK;  // empty caches: nothing to read
  if (!q_dev || !k_dev || !v_dev || !o_part_dev || !lse_part_dev)
    return fail(TC_ERR_INVALID_ARGUMENT, "null tensor pointer");
  if (!aligned16(q_dev) || !aligned16(k_dev) || !aligned16(v_dev) || !aligned16(o_part_dev))
    return fail(TC_ERR_ALIGNMENT, "q/k/v/o_part base pointers must be 16-byte aligned");
  if ((rc = check_strides("q", q_strides, 3)) != TC_OK) return rc;
  if ((rc = check_strides("k", k_strides, 3)) != TC_OK) return rc;
  if ((rc = check_strides("v", v_strides, 3)) != TC_OK) return rc;
  if (n_tokens < 0) return fail(TC_ERR_INVALID_ARGUMENT, "n_tokens %lld is negative", (long long)n_tokens);
  if (n_tokens > kMaxTokens)
    return fail(TC_ERR_INVALID_ARGUMENT, "n_tokens %lld above %lld", (long long)n_tokens, (long long)kMaxTokens);
  if (split_tokens <= 0 || split_tokens % kSplitGranule != 0)
    return fail(TC_ERR_INVALID_ARGUMENT, "split_tokens %d must be a positive multiple of %d", split_tokens,
                kSplitGranule);
  if (num_splits < 0 || num_splits > TC_MAX_SPLITS)
    return fail(TC_ERR_INVALID_ARGUMENT, "num_splits %d outside [0, %d]", num_splits, TC_MAX_SPLITS);
  if (static_cast<int64_t>(num_splits) * split_tokens < n_tokens)
    return fail(TC_ERR_INVALID_ARGUMENT, "%d splits of %d tokens do not cover %lld tokens", num_splits, split_tokens,
                (long long)n_tokens);
  if (static_cast<int64_t>(num_splits) * split_tokens > 2 * kMaxTokens)
    return fail(TC_ERR_INVALID_ARGUMENT, "%d splits of %d tokens span more than %lld tokens", num_splits,
                split_tokens, (long long)(2 * kMaxTokens));
  if (num_splits == 0) return TC_OK;
  if (!isfinite(scale)) return fail(TC_ERR_INVALID_ARGUMENT, "scale is not finite");
  // Per-lane buffer offsets span 16 token rows in 32 bits.
  constexpr int64_t kMaxTokenStride = int64_t(1) << 26;
  if (k_strides[2] < head_dim || v_strides[2] < head_dim || k_strides[2] >= kMaxTokenStride ||
      v_strides[2] >= kMaxTokenStride)
    return fail(TC_ERR_INVALID_ARGUMENT, "k/v token strides (%lld, %lld) outside [%d, 2^26)",
                (long long)k_strides[2], (long long)v_strides[2], head_dim);

  PartialArgs a;
  a.q = static_cast<const uint16_t*>(q_dev);
  a.k = static_cast<const uint16_t*>(k_dev);
  a.v = static_cast<const uint16_t*>(v_dev);
  a.o_part = o_part_dev;
  a.lse_part = lse_part_dev;
  a.lens = lens_dev;
  a.n = n_tokens;
  a.sq_b = q_strides[0]; a.sq_h = q_strides[1]; a.sq_g = q_strides[2];
  a.sk_b = k_strides[0]; a.sk_h = k_strides[1]; a.sk_t = k_strides[2];
  a.sv_b = v_strides[0]; a.sv_h = v_strides[1]; a.sv_t = v_strides[2];
  a.heads = kv_heads;
  a.group = group;
  a.splits = num_splits;
  a.split_tokens = split_tokens;
  a.interleave = interleave;
  // Longest sequences first: only for per-sequence lengths of a contiguous
  // cache, and up to 64 sequences (one lane each).
  a.longest_first = (lens_dev && !paged && batch > 1 && batch <= 64) ? 1 : 0;
  a.k_new = app ? static_cast<const uint16_t*>(app->k_new) : nullptr;
  a.v_new = app ? static_cast<const uint16_t*>(app->v_new) : nullptr;
  a.skn_b = app ? app->kn_strides[0] : 0;
  a.skn_h = app ? app->kn_strides[1] : 0;
  a.svn_b = app ? app->vn_strides[0] : 0;
  a.svn_h = app ? app->vn_strides[1] : 0;
  a.k_w = app ? static_cast<uint16_t*>(app->k_cache) : nullptr;
  a.v_w = app ? static_cast<uint16_t*>(app->v_cache) : nullptr;
  a.scale_log2 = static_cast<float>(static_cast<double>(scale) * 1.4426950408889634);
  a.tile_tab = paged ? paged->tile_tab : nullptr;
  a.tiles = paged ? paged->tiles : nullptr;
  a.max_tiles = paged ? paged->max_tiles : 0;
  a.pages = paged ? paged->pages : 0;
  a.page_tokens = paged ? paged->page_tokens : 0;
  a.tok_off = paged ? paged->tok_off : nullptr;
  a.tok_pitch = paged ? paged->tok_pitch : 0;
#if TC_DECODE_STAMPS
  a.stamps = g_stamps;
#endif

  hipStream_t s = static_cast<hipStream_t>(stream);
  const int waves = partial_waves(n_tokens, lens_dev != nullptr, paged != nullptr, app != nullptr, interleave);
  const hipError_t e = dtype == TC_DTYPE_F16 ? launch_partial_dt<TC_DTYPE_F16>(a, batch, waves, s)
                                             : launch_partial_dt<TC_DTYPE_BF16>(a, batch, waves, s);
  return hip_status(e, "decode_partial launch");
}

}  // namespace
}  // namespace tc

extern "C" {

int tc_decode_partial(const void* q_dev, const int64_t q_strides[3], const void* k_dev, const int64_t k_strides[3],
                      const void* v_dev, const int64_t v_strides[3], const int32_t* lens_dev, int64_t n_tokens,
                      int batch, int kv_heads, int group, int head_dim, int dtype, float scale, int split_tokens,
                      int num_splits, float* o_part_dev, float* lse_part_dev, void* stream) {
  clear_error();
  return partial_impl(q_dev, q_strides, k_dev, k_strides, v_dev, v_strides, lens_dev, n_tokens, batch, kv_heads, group,
                      head_dim, dtype, scale, split_tokens, num_splits, o_part_dev, lse_part_dev, 0, nullptr,
                      stream);
}

int tc_decode_partial_interleaved(const void* q_dev, const int64_t q_strides[3], const void* k_dev,
                                  const int64_t k_strides[3], const void* v_dev, const int64_t v_strides[3],
                                  const int32_t* lens_dev, int64_t n_tokens, int batch, int kv_heads, int group,
                                  int head_dim, int dtype, float scale, int split_tokens, int num_splits,
                                  float* o_part_dev, float* lse_part_dev, void* stream) {
  clear_error();
  return partial_impl(q_dev, q_strides, k_dev, k_strides, v_dev, v_strides, lens_dev, n_tokens, batch, kv_heads, group,
                      head_dim, dtype, scale, split_tokens, num_splits, o_part_dev, lse_part_dev, 1, nullptr,
                      stream);
}

int tc_decode_combine(const float* o_part_dev, const float* lse_part_dev, int batch, int kv_heads, int group,
                      int head_dim, int num_splits, void* out_dev, const int64_t out_strides[3], int dtype,
                      void* stream) {
  clear_error();
  int rc = check_common(batch, kv_heads, group, head_dim, dtype);
  if (rc != TC_OK) return rc;
  if (!out_dev || (num_splits > 0 && (!o_part_dev || !lse_part_dev)))
    return fail(TC_ERR_INVALID_ARGUMENT, "null tensor pointer");
  if (!aligned16(out_dev) || (num_splits > 0 && !aligned16(o_part_dev)))
    return fail(TC_ERR_ALIGNMENT, "out/o_part base pointers must be 16-byte aligned");
  if ((rc = check_strides("out", out_strides, 3)) != TC_OK) return rc;
  if (num_splits < 0 || num_splits > TC_MAX_SPLITS)
    return fail(TC_ERR_INVALID_ARGUMENT, "num_splits %d outside [0, %d]", num_splits, TC_MAX_SPLITS);

  CombineArgs a;
  a.o_part = o_part_dev;
  a.lse_part = lse_part_dev;
  a.out = static_cast<uint16_t*>(out_dev);
  a.so_b = out_strides[0]; a.so_h = out_strides[1]; a.so_g = out_strides[2];
  a.heads = kv_heads;
  a.group = group;
  a.splits = num_splits;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // One wave per (KV head, sequence, query head, quarter of the dims), the KV
  // head fastest.
  const dim3 grid(kv_heads, batch, group * 4), block(64);
  if (dtype == TC_DTYPE_F16)
    hipLaunchKernelGGL((decode_combine_kernel<TC_DTYPE_F16>), grid, block, 0, s, a);
  else
    hipLaunchKernelGGL((decode_combine_kernel<TC_DTYPE_BF16>), grid, block, 0, s, a);
  return hip_status(hipGetLastError(), "decode_combine launch");
}

}  // extern "C"

namespace tc {
namespace {

int attention_impl(const void* q_dev, const int64_t q_strides[3], const void* k_dev, const int64_t k_strides[3],
                   const void* v_dev, const int64_t v_strides[3], const int32_t* lens_dev, int64_t n_tokens,
                   int batch, int kv_heads, int group, int head_dim, int dtype, float scale, int split_tokens,
                   void* workspace_dev, size_t workspace_bytes, void* out_dev, const int64_t out_strides[3],
                   const Append* app, int ragged_plan, void* stream, const Paged* paged = nullptr) {
  int rc = check_common(batch, kv_heads, group, head_dim, dtype);
  if (rc != TC_OK) return rc;
  if (n_tokens < 0) return fail(TC_ERR_INVALID_ARGUMENT, "n_tokens %lld is negative", (long long)n_tokens);
  int S = 0, t = 0;
  if ((rc = split_plan(batch, kv_heads, n_tokens, split_tokens, ragged_plan, &S, &t)) != TC_OK) return rc;
  const size_t need = tc_decode_workspace_bytes(batch, kv_heads, group, head_dim, S);
  if (S > 0 && (!workspace_dev || workspace_bytes < need))
    return fail(TC_ERR_WORKSPACE, "workspace of %zu bytes, %zu needed for %d splits", workspace_bytes, need, S);
  float* o_part = static_cast<float*>(workspace_dev);
  float* lse_part = S > 0 ? o_part + static_cast<size_t>(batch) * kv_heads * S * group * head_dim : nullptr;
  if (S > 0) {
    // Splits here are internal, so their tiles are dealt round-robin (the merged result is the same).
    rc = partial_impl(q_dev, q_strides, k_dev, k_strides, v_dev, v_strides, lens_dev, n_tokens, batch, kv_heads, group,
                      head_dim, dtype, scale, t, S, o_part, lse_part, TC_DECODE_INTERLEAVE, app, stream, paged);
    if (rc != TC_OK) return rc;
  }
  return tc_decode_combine(o_part, lse_part, batch, kv_heads, group, head_dim, S, out_dev, out_strides, dtype, stream);
}

}  // namespace
}  // namespace tc

extern "C" {

int tc_decode_attention(const void* q_dev, const int64_t q_strides[3], const void* k_dev, const int64_t k_strides[3],
                        const void* v_dev, const int64_t v_strides[3], const int32_t* lens_dev, int64_t n_tokens,
                        int batch, int kv_heads, int group, int head_dim, int dtype, float scale, int split_tokens,
                        void* workspace_dev, size_t workspace_bytes, void* out_dev, const int64_t out_strides[3],
                        void* stream) {
  clear_error();
  return attention_impl(q_dev, q_strides, k_dev, k_strides, v_dev, v_strides, lens_dev, n_tokens, batch, kv_heads,
                        group, head_dim, dtype, scale, split_tokens, workspace_dev, workspace_bytes, out_dev,
                        out_strides, nullptr, lens_dev != nullptr, stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free decode: the split partials of tc_decode_attention_noalloc
// live in `scratch`, a static array that every GPU the library runs on holds
// until the process ends. Its device address differs per GPU and is taken
// once per device with hipGetSymbolAddress; host code never passes the
// array's own name to a kernel.
// ---------------------------------------------------------------------------

static __device__ __align__(256) unsigned char scratch[TC_DECODE_SCRATCH_BYTES];

namespace tc {
namespace {

constexpr int kScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_dev[kScratchDevices] = {};

// Device address of `scratch` on the current device (looked up on first use).
int scratch_on_current_device(void** out) {
  int dev = 0;
  int rc = hip_status(hipGetDevice(&dev), "hipGetDevice");
  if (rc != TC_OK) return rc;
  if (dev < 0 || dev >= kScratchDevices) return fail(TC_ERR_HIP, "device id %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (!g_scratch_dev[dev]) {
    void* p = nullptr;
    rc = hip_status(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (rc != TC_OK) return rc;
    if (!p || !aligned16(p)) return fail(TC_ERR_HIP, "scratch symbol address %p unusable", p);
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return TC_OK;
}

}  // namespace
}  // namespace tc

extern "C" {

int tc_decode_attention_noalloc(const void* q_dev, const int64_t q_strides[3], const void* k_dev,
                                const int64_t k_strides[3], const void* v_dev, const int64_t v_strides[3],
                                const int32_t* lens_dev, int64_t n_tokens, int batch, int kv_heads, int group,
                                int head_dim, int dtype, float scale, int split_tokens, void* out_dev,
                                const int64_t out_strides[3], void* stream) {
  clear_error();
  int rc = check_common(batch, kv_heads, group, head_dim, dtype);
  if (rc != TC_OK) return rc;
  if (n_tokens < 0) return fail(TC_ERR_INVALID_ARGUMENT, "n_tokens %lld is negative", (long long)n_tokens);
  int S = 0, t = 0;
  if ((rc = split_plan(batch, kv_heads, n_tokens, split_tokens, lens_dev != nullptr, &S, &t)) != TC_OK) return rc;
  const size_t need = tc_decode_workspace_bytes(batch, kv_heads, group, head_dim, S);
  if (need > TC_DECODE_SCRATCH_BYTES)
    return fail(TC_ERR_WORKSPACE,
                "%d splits of batch %d x %d kv heads x %d query heads need %zu bytes of partials; the static scratch "
                "holds %zu (pass a workspace to tc_decode_attention instead)",
                S, batch, kv_heads, group, need, (size_t)TC_DECODE_SCRATCH_BYTES);
  void* ws = nullptr;
  if (S > 0 && (rc = scratch_on_current_device(&ws)) != TC_OK) return rc;
  return attention_impl(q_dev, q_strides, k_dev, k_strides, v_dev, v_strides, lens_dev, n_tokens, batch, kv_heads,
                        group, head_dim, dtype, scale, split_tokens, ws, TC_DECODE_SCRATCH_BYTES, out_dev,
                        out_strides, nullptr, lens_dev != nullptr, stream);
}

static int append_impl(const void* q_dev, const int64_t q_strides[3], void* k_cache_dev, const int64_t k_strides[3],
                       void* v_cache_dev, const int64_t v_strides[3], const void* k_new_dev,
                       const int64_t k_new_strides[2], const void* v_new_dev, const int64_t v_new_strides[2],
                       const int32_t* pos_dev, int64_t n_tokens, int batch, int kv_heads, int group, int head_dim,
                       int dtype, float scale, int split_tokens, void* workspace_dev, size_t workspace_bytes,
                       void* out_dev, const int64_t out_strides[3], void* stream) {
  if (n_tokens < 1) return fail(TC_ERR_INVALID_ARGUMENT, "append needs n_tokens >= 1 (got %lld)", (long long)n_tokens);
  if (!k_new_dev || !v_new_dev || !k_new_strides || !v_new_strides)
    return fail(TC_ERR_INVALID_ARGUMENT, "null new-token K/V");
  if (!aligned16(k_new_dev) || !aligned16(v_new_dev))
    return fail(TC_ERR_ALIGNMENT, "new-token K/V not 16-byte aligned");
  for (int i = 0; i < 2; ++i)
    if (k_new_strides[i] < 0 || v_new_strides[i] < 0 || k_new_strides[i] % 8 || v_new_strides[i] % 8)
      return fail(TC_ERR_ALIGNMENT, "new-token K/V strides must be non-negative multiples of 8");
  const Append app{k_new_dev, k_new_strides, v_new_dev, v_new_strides, k_cache_dev, v_cache_dev};
  return attention_impl(q_dev, q_strides, k_cache_dev, k_strides, v_cache_dev, v_strides, pos_dev, n_tokens, batch,
                        kv_heads, group, head_dim, dtype, scale, split_tokens, workspace_dev, workspace_bytes, out_dev,
                        out_strides, &app, 0, stream);
}

int tc_decode_append_attention(const void* q_dev, const int64_t q_strides[3], void* k_cache_dev,
                               const int64_t k_strides[3], void* v_cache_dev, const int64_t v_strides[3],
                               const void* k_new_dev, const int64_t k_new_strides[2], const void* v_new_dev,
                               const int64_t v_new_strides[2], int64_t n_tokens, int batch, int kv_heads, int group,
                               int head_dim, int dtype, float scale, int split_tokens, void* workspace_dev,
                               size_t workspace_bytes, void* out_dev, const int64_t out_strides[3], void* stream) {
  clear_error();
  return append_impl(q_dev, q_strides, k_cache_dev, k_strides, v_cache_dev, v_strides, k_new_dev, k_new_strides,
                     v_new_dev, v_new_strides, nullptr, n_tokens, batch, kv_heads, group, head_dim, dtype, scale,
                     split_tokens, workspace_dev, workspace_bytes, out_dev, out_strides, stream);
}

int tc_decode_append_attention_at(const void* q_dev, const int64_t q_strides[3], void* k_cache_dev,
                                  const int64_t k_strides[3], void* v_cache_dev, const int64_t v_strides[3],
                                  const void* k_new_dev, const int64_t k_new_strides[2], const void* v_new_dev,
                                  const int64_t v_new_strides[2], const int32_t* pos_dev, int64_t capacity,
                                  int batch, int kv_heads, int group, int head_dim, int dtype, float scale,
                                  int split_tokens, void* workspace_dev, size_t workspace_bytes, void* out_dev,
                                  const int64_t out_strides[3], void* stream) {
  clear_error();
  if (!pos_dev) return fail(TC_ERR_INVALID_ARGUMENT, "null append positions");
  return append_impl(q_dev, q_strides, k_cache_dev, k_strides, v_cache_dev, v_strides, k_new_dev, k_new_strides,
                     v_new_dev, v_new_strides, pos_dev, capacity, batch, kv_heads, group, head_dim, dtype, scale,
                     split_tokens, workspace_dev, workspace_bytes, out_dev, out_strides, stream);
}

int tc_decode_paged_attention(const void* q_dev, const int64_t q_strides[3], const void* k_pool_dev,
                              const void* v_pool_dev, const int64_t pool_strides[3], int num_pages, int page_tokens,
                              const int32_t* tile_table_dev, const int32_t* tiles_dev, int64_t max_tiles, int batch,
                              int kv_heads, int group, int head_dim, int dtype, float scale, int split_tokens,
                              void* workspace_dev, size_t workspace_bytes, void* out_dev,
                              const int64_t out_strides[3], void* stream) {
  clear_error();
  if (num_pages < 1 || page_tokens < 1)
    return fail(TC_ERR_INVALID_ARGUMENT, "pool of %d pages of %d tokens", num_pages, page_tokens);
  if (max_tiles < 0 || max_tiles > kMaxTokens / 16)
    return fail(TC_ERR_INVALID_ARGUMENT, "max_tiles %lld outside [0, %lld]", (long long)max_tiles,
                (long long)(kMaxTokens / 16));
  if (max_tiles > 0 && (!tile_table_dev || !tiles_dev)) return fail(TC_ERR_INVALID_ARGUMENT, "null tile table");
  if (max_tiles > 0 && !aligned16(tile_table_dev))
    return fail(TC_ERR_ALIGNMENT, "tile table not 16-byte aligned");
  if (!pool_strides) return fail(TC_ERR_INVALID_ARGUMENT, "null pool strides");
  // An empty table plans zero splits, so the partial kernel (the only reader
  // of the table) is not launched.
  const Paged p{tile_table_dev, tiles_dev, max_tiles, num_pages, page_tokens};
  return attention_impl(q_dev, q_strides, k_pool_dev, pool_strides, v_pool_dev, pool_strides, nullptr,
                        16 * max_tiles, batch, kv_heads, group, head_dim, dtype, scale, split_tokens, workspace_dev,
                        workspace_bytes, out_dev, out_strides, nullptr, batch > 1, stream, &p);
}

int tc_decode_paged_append_attention(const void* q_dev, const int64_t q_strides[3], void* k_pool_dev,
                                     void* v_pool_dev, const int64_t pool_strides[3], int num_pages,
                                     int page_tokens, const int32_t* tile_table_dev, const int32_t* tiles_dev,
                                     int64_t max_tiles, const void* k_new_dev, const int64_t k_new_strides[2],
                                     const void* v_new_dev, const int64_t v_new_strides[2], int batch,
                                     int kv_heads, int group, int head_dim, int dtype, float scale,
                                     int split_tokens, void* workspace_dev, size_t workspace_bytes, void* out_dev,
                                     const int64_t out_strides[3], void* stream) {
  clear_error();
  if (num_pages < 1 || page_tokens < 1)
    return fail(TC_ERR_INVALID_ARGUMENT, "pool of %d pages of %d tokens", num_pages, page_tokens);
  if (max_tiles < 1 || max_tiles > kMaxTokens / 16)
    return fail(TC_ERR_INVALID_ARGUMENT, "append needs max_tiles in [1, %lld] (got %lld)",
                (long long)(kMaxTokens / 16), (long long)max_tiles);
  if (!tile_table_dev || !tiles_dev) return fail(TC_ERR_INVALID_ARGUMENT, "null tile table");
  if (!aligned16(tile_table_dev)) return fail(TC_ERR_ALIGNMENT, "tile table not 16-byte aligned");
  if (!pool_strides) return fail(TC_ERR_INVALID_ARGUMENT, "null pool strides");
  if (!k_new_dev || !v_new_dev || !k_new_strides || !v_new_strides)
    return fail(TC_ERR_INVALID_ARGUMENT, "null new-token K/V");
  if (!aligned16(k_new_dev) || !aligned16(v_new_dev))
    return fail(TC_ERR_ALIGNMENT, "new-token K/V not 16-byte aligned");
  for (int i = 0; i < 2; ++i)
    if (k_new_strides[i] < 0 || v_new_strides[i] < 0 || k_new_strides[i] % 8 || v_new_strides[i] % 8)
      return fail(TC_ERR_ALIGNMENT, "new-token K/V strides must be non-negative multiples of 8");
  const Append app{k_new_dev, k_new_strides, v_new_dev, v_new_strides, k_pool_dev, v_pool_dev};
  const Paged p{tile_table_dev, tiles_dev, max_tiles, num_pages, page_tokens};
  return attention_impl(q_dev, q_strides, k_pool_dev, pool_strides, v_pool_dev, pool_strides, nullptr,
                        16 * max_tiles, batch, kv_heads, group, head_dim, dtype, scale, split_tokens, workspace_dev,
                        workspace_bytes, out_dev, out_strides, &app, batch > 1, stream, &p);
}

int tc_decode_paged_append_attention_at(const void* q_dev, const int64_t q_strides[3], void* k_pool_dev,
                                        void* v_pool_dev, const int64_t pool_strides[3], int num_pages,
                                        int page_tokens, const int32_t* tile_table_dev, const int32_t* tiles_dev,
                                        int64_t max_tiles, const int32_t* tok_off_dev, int64_t tok_pitch,
                                        const int32_t* lens_dev, const void* k_new_dev,
                                        const int64_t k_new_strides[2], const void* v_new_dev,
                                        const int64_t v_new_strides[2], int batch, int kv_heads, int group,
                                        int head_dim, int dtype, float scale, int split_tokens, void* workspace_dev,
                                        size_t workspace_bytes, void* out_dev, const int64_t out_strides[3],
                                        void* stream) {
  clear_error();
  if (num_pages < 1 || page_tokens < 1)
    return fail(TC_ERR_INVALID_ARGUMENT, "pool of %d pages of %d tokens", num_pages, page_tokens);
  if (max_tiles < 1 || max_tiles > kMaxTokens / 16)
    return fail(TC_ERR_INVALID_ARGUMENT, "append needs max_tiles in [1, %lld] (got %lld)",
                (long long)(kMaxTokens / 16), (long long)max_tiles);
  if (!tile_table_dev || !tiles_dev || !tok_off_dev || !lens_dev)
    return fail(TC_ERR_INVALID_ARGUMENT, "null tile table, token offsets or lengths");
  if (!aligned16(tile_table_dev)) return fail(TC_ERR_ALIGNMENT, "tile table not 16-byte aligned");
  if (tok_pitch < 1 || tok_pitch > kMaxTokens)
    return fail(TC_ERR_INVALID_ARGUMENT, "token offset rows of %lld entries", (long long)tok_pitch);
  if (!pool_strides) return fail(TC_ERR_INVALID_ARGUMENT, "null pool strides");
  if (static_cast<int64_t>(num_pages) * pool_strides[0] * 2 >= (int64_t(1) << 31))
    return fail(TC_ERR_UNSUPPORTED, "pools of 2 GiB or more (token offsets are 32-bit)");
  if (!k_new_dev || !v_new_dev || !k_new_strides || !v_new_strides)
    return fail(TC_ERR_INVALID_ARGUMENT, "null new-token K/V");
  if (!aligned16(k_new_dev) || !aligned16(v_new_dev))
    return fail(TC_ERR_ALIGNMENT, "new-token K/V not 16-byte aligned");
  for (int i = 0; i < 2; ++i)
    if (k_new_strides[i] < 0 || v_new_strides[i] < 0 || k_new_strides[i] % 8 || v_new_strides[i] % 8)
      return fail(TC_ERR_ALIGNMENT, "new-token K/V strides must be non-negative multiples of 8");
  const Append app{k_new_dev, k_new_strides, v_new_dev, v_new_strides, k_pool_dev, v_pool_dev};
  const Paged p{tile_table_dev, tiles_dev, max_tiles, num_pages, page_tokens, tok_off_dev, tok_pitch};
  return attention_impl(q_dev, q_strides, k_pool_dev, pool_strides, v_pool_dev, pool_strides, lens_dev,
                        16 * max_tiles, batch, kv_heads, group, head_dim, dtype, scale, split_tokens, workspace_dev,
                        workspace_bytes, out_dev, out_strides, &app, batch > 1, stream, &p);
}

}  // extern "C"

#if TC_DECODE_STAMPS
// Measurement build only (libthreadcut_stamps.so): the device buffer that the
// partial kernels launched from now on record their wave timelines into
// (8 words per wave, see PartialArgs::stamps), or null for none.
extern "C" void tc_decode_set_stamps(void* stamps_dev) { tc::g_stamps = static_cast<unsigned long long*>(stamps_dev); }
#endif
