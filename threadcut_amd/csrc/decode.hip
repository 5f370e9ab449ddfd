// Split-KV GQA flash-decode for gfx950: a partial online-softmax kernel over
// (split, kv head, sequence) work-groups and a separate log-sum-exp combine.
//
// Reference semantics: threadcut/flash_decode.py:21-54 (`_partial`: fp32
// math, scale applied after q.k, -inf guards, out = acc / l, lse = m + log l)
// and :57-69 (decode_attention: splits = cdiv(n, split), merge with
// softmax(lse) weights, cast to q.dtype).
//
// Layout of one wave64 over the cache: a 16-token iteration issues four
// 1 KiB-contiguous 128-bit loads of K (and four of V). Lane l reads token
// t0 + 4j + (l >> 4), dims 8*(l & 15) .. +8, for j = 0..3, so the wave's 16
// lanes of a row hold one token and the four rows hold four tokens. The g
// query heads of the KV head stay in registers and share every K/V element.
//   - q.k: v_dot2_f32_{f16,bf16} over the lane's 8 dims, then a DPP
//     reduce-scatter inside each row (4 steps) leaves every lane with the full
//     score of one (token, head) pair (two for g > 4);
//   - online softmax per row and head in the log2 domain (exp2), max via two
//     DPP steps over the four lanes of a head;
//   - p.v: each lane accumulates its 8 dims for the row's token, p broadcast
//     from the owning lane with DPP row_newbcast.
// Four rows x four waves are independent online-softmax streams; they are
// merged once at the end (cross-row shuffles, then LDS across waves) so each
// work-group writes one (o, lse) partial per query head.
#include <math.h>

#include <algorithm>

#include "tc_common.hpp"

namespace tc {
namespace {

// Tuning knobs (measured on MI355X; override with -D for sweeps).
#ifndef TC_DECODE_WAVES
#define TC_DECODE_WAVES 4   // waves per partial work-group
#endif
#ifndef TC_DECODE_DEPTH
#define TC_DECODE_DEPTH 2   // 16-token tiles in flight per wave
#endif
#ifndef TC_DECODE_AUX
#define TC_DECODE_AUX 2     // cache-policy bits of the K/V buffer loads (2: non-temporal stream)
#endif
#ifndef TC_DECODE_PERMLANE
#define TC_DECODE_PERMLANE 1  // merge the four rows of a wave with v_permlane{16,32}_swap
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

constexpr int kHeadDim = 128;
constexpr int64_t kMaxTokens = int64_t(1) << 29;  // token positions stay 32-bit in the kernel
constexpr int kWaves = TC_DECODE_WAVES;
constexpr int kDepth = TC_DECODE_DEPTH;
constexpr int kWaveIter = 16;                        // tokens per wave iteration
constexpr int kSplitGranule = kWaves * kWaveIter > 64 ? kWaves * kWaveIter : 64;  // split length granule
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
  float scale_log2;    // softmax scale * log2(e)
  // Append (k_new != null): the cache holds n - 1 tokens and the new token's
  // K/V rows [B, H, D] are attended from k_new/v_new and written to row n - 1
  // of the cache (k_w/v_w) by wave 0 of split 0; no other wave reads that row.
  const uint16_t* k_new;
  const uint16_t* v_new;
  int64_t skn_b, skn_h, svn_b, svn_h;
  uint16_t* k_w;
  uint16_t* v_w;
};

struct CombineArgs {
  const float* o_part;
  const float* lse_part;
  uint16_t* out;
  int64_t so_b, so_h, so_g;
  int heads, group, splits;
};

__device__ __forceinline__ uint4 load16(const uint16_t* p) {
  return *reinterpret_cast<const uint4*>(p);
}

__device__ __forceinline__ uint32_t word(const uint4& x, int i) {
  return i == 0 ? x.x : (i == 1 ? x.y : (i == 2 ? x.z : x.w));
}

// Lane permutations that make the row reduction select-free.
//
// A lane's partial dots are x[slot' * GP + head'] (slot' < 4, head' < GP):
// K register slot' holds token slot slot' ^ (c >> 2) of the iteration and q
// register head' holds query row head' ^ head_perm(c). Written as a bit
// vector, register r of lane c then carries value r ^ X(c), where X is the
// linear map that sends the DPP partner patterns used below (c ^ 8, c ^ 7
// via half-mirror, c ^ 2, c ^ 1) to the register bits halved at each step.
// Every step is x[i] += dpp(x[i + K/2]) on all lanes: no per-lane selects.
template <int GP>
__device__ __forceinline__ int head_perm(int c) {
  const int flip = ((c >> 2) & 1) ? 3 : 0;
  if constexpr (GP == 1) return 0;
  else if constexpr (GP == 2) return ((c >> 1) & 1) ^ ((c >> 2) & 1);
  else if constexpr (GP == 4) return (c & 3) ^ flip;
  else return 2 * ((c & 3) ^ flip);
}

// Row lane holding the score of (token slot j, head hh) after the scatter.
template <int GP>
constexpr int owner_lane(int j, int hh) {
  return GP == 1 ? 4 * j
       : GP == 2 ? 4 * j + 2 * (hh ^ (j & 1))
       : GP == 4 ? 4 * j + (hh ^ ((j & 1) ? 3 : 0))
                 : 4 * j + ((hh >> 1) ^ ((j & 1) ? 3 : 0));
}

// Register (index < VPL) of that lane holding it.
template <int GP>
constexpr int owner_reg(int hh) { return GP == 8 ? (hh & 1) : 0; }

// Sum of the NV = 4 * GP partial dots over the 16 lanes of each row,
// scattered: lane c keeps the totals of its first VPL registers.
template <int NV>
__device__ __forceinline__ void row_reduce_scatter(float* x) {
#pragma unroll
  for (int i = 0; i < NV / 2; ++i) x[i] += dpp<DPP_ROW_ROR8>(x[i + NV / 2]);
#pragma unroll
  for (int i = 0; i < NV / 4; ++i) x[i] += dpp<DPP_ROW_HALF_MIRROR>(x[i + NV / 4]);
  if constexpr (NV / 8 >= 1) {
#pragma unroll
    for (int i = 0; i < NV / 8; ++i) x[i] += dpp<DPP_QUAD_XOR2>(x[i + NV / 8]);
  } else {
    x[0] += dpp<DPP_QUAD_XOR2>(x[0]);
  }
  if constexpr (NV / 16 >= 1) {
#pragma unroll
    for (int i = 0; i < NV / 16; ++i) x[i] += dpp<DPP_QUAD_XOR1>(x[i + NV / 16]);
  } else {
    x[0] += dpp<DPP_QUAD_XOR1>(x[0]);
  }
}

// All-reduce over the four lanes of a row that own one head (c, c^8, c^7, c^15).
__device__ __forceinline__ float head_max(float t) {
  t = fmaxf(t, dpp<DPP_ROW_ROR8>(t));
  return fmaxf(t, dpp<DPP_ROW_HALF_MIRROR>(t));
}
__device__ __forceinline__ float head_sum(float t) {
  t += dpp<DPP_ROW_ROR8>(t);
  return t + dpp<DPP_ROW_HALF_MIRROR>(t);
}

// Value of x held by lane k of the caller's row; k folds to a constant after
// unrolling, so the switch reduces to one DPP move.
__device__ __forceinline__ float row_bcast_dyn(float x, int k) {
  switch (k) {
    case 0: return row_bcast<0>(x);
    case 1: return row_bcast<1>(x);
    case 2: return row_bcast<2>(x);
    case 3: return row_bcast<3>(x);
    case 4: return row_bcast<4>(x);
    case 5: return row_bcast<5>(x);
    case 6: return row_bcast<6>(x);
    case 7: return row_bcast<7>(x);
    case 8: return row_bcast<8>(x);
    case 9: return row_bcast<9>(x);
    case 10: return row_bcast<10>(x);
    case 11: return row_bcast<11>(x);
    case 12: return row_bcast<12>(x);
    case 13: return row_bcast<13>(x);
    case 14: return row_bcast<14>(x);
    default: return row_bcast<15>(x);
  }
}

template <int GP>
__device__ __forceinline__ float owner_bcast(const float* x, int j, int hh) {
  return row_bcast_dyn(x[owner_reg<GP>(hh)], owner_lane<GP>(j, hh));
}

// Reductions over the four 16-lane rows of a wave (every lane gets the result).
#if TC_DECODE_PERMLANE
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
#else
__device__ __forceinline__ float rows_sum(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}
__device__ __forceinline__ float rows_max(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}
#endif

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Buffer resource over `bytes` bytes at p; loads past the end return zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, int32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, 0x00020000);
}

__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, int32_t off) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, TC_DECODE_AUX);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// K/V rows of one 16-token iteration of a wave: rows at or past `end` read
// as zero (their scores are masked), so no index clamping is needed.
struct Tile {
  uint4 k[4];  // register j: token slot j ^ (c >> 2)
  uint4 v[4];  // register j: token slot j
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

template <int DT, int GP>
struct Stream {
  static constexpr int NV = 4 * GP;                   // partial dots per lane per iteration
  static constexpr int VPL = NV >= 16 ? NV / 16 : 1;  // scores owned per lane
  float m[VPL];          // running max (log2 domain) of the lane's head(s), per row
  float l[VPL];          // running sum of exp2(score - m) over the lane's token slot
  float acc[GP][8];      // running p.v for the lane's 8 dims, every head

  __device__ __forceinline__ void init() {
#pragma unroll
    for (int i = 0; i < VPL; ++i) { m[i] = neg_inf(); l[i] = 0.f; }
#pragma unroll
    for (int hh = 0; hh < GP; ++hh)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[hh][e] = 0.f;
  }

  // One 16-token iteration; `valid` masks the lane's score(s).
  __device__ __forceinline__ void step(const Tile& t, const uint32_t (&qw)[GP][4], bool valid, float scale_log2) {
    using E = Elem<DT>;
    float x[NV];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int hh = 0; hh < GP; ++hh) {
        float d = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) d = E::dot2(word(t.k[j], w), qw[hh][w], d);
        x[j * GP + hh] = d;
      }
    row_reduce_scatter<NV>(x);

    float p[VPL], alpha[VPL];
    bool rescale = false;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const float s = valid ? x[i] * scale_log2 : neg_inf();
      const float mn = fmaxf(m[i], head_max(s));
      const float ms = (mn == neg_inf()) ? 0.f : mn;
      p[i] = __builtin_amdgcn_exp2f(s - ms);
      alpha[i] = __builtin_amdgcn_exp2f(m[i] - ms);
      rescale |= (mn != m[i]) && (m[i] != neg_inf());
      l[i] = l[i] * alpha[i] + p[i];
      m[i] = mn;
    }
    if (__any(rescale)) {
#pragma unroll
      for (int hh = 0; hh < GP; ++hh) {
        const float ah = owner_bcast<GP>(alpha, 0, hh);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[hh][e] *= ah;
      }
    }

#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float vf[8];
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        vf[2 * w] = E::lo(word(t.v[j], w));
        vf[2 * w + 1] = E::hi(word(t.v[j], w));
      }
#pragma unroll
      for (int hh = 0; hh < GP; ++hh) {
        const float pj = owner_bcast<GP>(p, j, hh);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[hh][e] = fmaf(pj, vf[e], acc[hh][e]);
      }
    }
  }
};

template <int DT, int GP>
__global__ __launch_bounds__(64 * kWaves) void decode_partial_kernel(const PartialArgs a) {
  __shared__ float s_acc[kWaves][GP][kHeadDim];
  __shared__ float s_m[kWaves][GP];
  __shared__ float s_l[kWaves][GP];

  const int lane = threadIdx.x & 63;
  // Wave-uniform by construction; readfirstlane lets the compiler keep the
  // token range (and so the buffer resources) in scalar registers.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = lane >> 4;
  const int c = lane & 15;
  const int split = blockIdx.x;
  const int h = blockIdx.y;
  const int b = blockIdx.z;

  // Cached tokens attended. Lengths past the buffer (or negative) are clamped
  // into [0, n]. With an append the new token is one more, read from
  // k_new/v_new and written to row `len`, so len stays below n: n - 1
  // without lengths, lens[b] (the append position) clamped to n - 1 with.
  // Token positions are 32-bit (the host keeps n and S * T below 2^30), and
  // nothing before the first K/V requests divides: every wave runs this
  // prologue before its first load, so its length is latency.
  const char* kslab = reinterpret_cast<const char*>(a.k + b * a.sk_b + h * a.sk_h);
  const char* vslab = reinterpret_cast<const char*>(a.v + b * a.sv_b + h * a.sv_h);
  const int32_t row_k = static_cast<int32_t>(a.sk_t) * 2, row_v = static_cast<int32_t>(a.sv_t) * 2;
  // Materialise the slab addresses here so their kernel arguments are fetched
  // with the others at entry (one scalar round trip instead of two).
  __asm__ volatile("" ::"s"(kslab), "s"(vslab));
  const int32_t n = static_cast<int32_t>(a.n);
  const int32_t len_cap = a.k_new ? n - 1 : n;
  int32_t len = len_cap;
  if (a.lens) len = min(max(a.lens[b], 0), len_cap);
  // The wave's 16-token tiles start at tok and advance by tok_step while
  // below end. Contiguous: split s, wave w own [s*T + w*T/W, s*T + (w+1)*T/W).
  // Interleaved: all S*W waves of a head sweep the cache together, wave g
  // taking tiles g, g + S*W, ..., so the loads in flight at any moment are
  // adjacent in HBM.
  int32_t tok, tok_step, end;
  if (a.interleave) {
    tok = (split * kWaves + wave) * kWaveIter;
    tok_step = a.splits * kWaves * kWaveIter;
    end = len;
  } else {
    const int32_t wave_tokens = a.split_tokens / kWaves;
    tok = split * a.split_tokens + wave * wave_tokens;
    tok_step = kWaveIter;
    end = min(tok + wave_tokens, len);
  }

  int32_t koff[4], voff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    koff[j] = (4 * (j ^ (c >> 2)) + grp) * row_k + 16 * c;
    voff[j] = (4 * j + grp) * row_v + 16 * c;
  }
  // Ring of kDepth tiles, the first kDepth - 1 requested before anything
  // else. Loads past `end` read nothing (the buffer range is empty there).
  Tile t[kDepth];
#pragma unroll
  for (int d = 0; d < kDepth - 1; ++d)
    load_tile(t[d], kslab, vslab, row_k, row_v, tok + d * tok_step, end, koff, voff);

  // The lane's 8 dims of every query row, in the lane's head order.
  uint32_t qw[GP][4];
  {
    const uint16_t* qb = a.q + b * a.sq_b + h * a.sq_h + 8 * c;
    const int hp = head_perm<GP>(c);
#pragma unroll
    for (int hh = 0; hh < GP; ++hh) {
      const int row = hh ^ hp;
      uint4 q4 = make_uint4(0u, 0u, 0u, 0u);
      if (row < a.group) q4 = *reinterpret_cast<const uint4*>(qb + row * a.sq_g);
      qw[hh][0] = q4.x; qw[hh][1] = q4.y; qw[hh][2] = q4.z; qw[hh][3] = q4.w;
    }
  }

  Stream<DT, GP> st;
  st.init();
  const int my_slot = 4 * (c >> 2) + grp;  // token slot of the lane's score(s)

  if (tok < end) {
    // Tile d of a round is computed while the next kDepth - 1 tiles are in
    // flight (ring indices fold to constants when unrolled).
    for (;;) {
      bool done = false;
#pragma unroll
      for (int d = 0; d < kDepth; ++d) {
        if (!done) {
          load_tile(t[(d + kDepth - 1) % kDepth], kslab, vslab, row_k, row_v, tok + (kDepth - 1) * tok_step, end,
                    koff, voff);
          st.step(t[d], qw, tok + my_slot < end, a.scale_log2);
          tok += tok_step;
          done = tok >= end;
        }
      }
      if (done) break;
    }
  }

  if (a.k_new && split == 0 && wave == 0) {
    // The appended token, as a tile whose only row is slot 0 (the buffer range
    // is one row, so the other slots read zero and are masked).
    const char* kn = reinterpret_cast<const char*>(a.k_new + b * a.skn_b + h * a.skn_h);
    const char* vn = reinterpret_cast<const char*>(a.v_new + b * a.svn_b + h * a.svn_h);
    const __amdgpu_buffer_rsrc_t rk = make_rsrc(kn, kHeadDim * 2);
    const __amdgpu_buffer_rsrc_t rv = make_rsrc(vn, kHeadDim * 2);
    Tile tn;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      tn.k[j] = bload16(rk, koff[j]);
      tn.v[j] = bload16(rv, voff[j]);
    }
    st.step(tn, qw, my_slot == 0, a.scale_log2);
    if (lane < 32) {
      const bool is_v = lane >= 16;
      const int chunk = 8 * (lane & 15);
      const uint16_t* src = is_v ? a.v_new + b * a.svn_b + h * a.svn_h : a.k_new + b * a.skn_b + h * a.skn_h;
      uint16_t* dst = is_v ? a.v_w + b * a.sv_b + h * a.sv_h + len * a.sv_t
                           : a.k_w + b * a.sk_b + h * a.sk_h + len * a.sk_t;
      *reinterpret_cast<uint4*>(dst + chunk) = *reinterpret_cast<const uint4*>(src + chunk);
    }
  }

  constexpr int VPL = Stream<DT, GP>::VPL;
  // Row totals of l over the four token slots of each head, then every
  // head's (m, l) to every lane.
#pragma unroll
  for (int i = 0; i < VPL; ++i) st.l[i] = head_sum(st.l[i]);
  float mh[GP], lh[GP];
#pragma unroll
  for (int hh = 0; hh < GP; ++hh) {
    mh[hh] = owner_bcast<GP>(st.m, 0, hh);
    lh[hh] = owner_bcast<GP>(st.l, 0, hh);
  }

  // Merge the four rows (lanes c, c+16, c+32, c+48 hold the same dims).
#pragma unroll
  for (int hh = 0; hh < GP; ++hh) {
    const float M = rows_max(mh[hh]);
    const float f = __builtin_amdgcn_exp2f(mh[hh] - ((M == neg_inf()) ? 0.f : M));
    lh[hh] = rows_sum(lh[hh] * f);
#pragma unroll
    for (int e = 0; e < 8; ++e) st.acc[hh][e] = rows_sum(st.acc[hh][e] * f);
    mh[hh] = M;
  }

  // Merge the waves through LDS and write this split's partial.
  if (grp == 0) {
#pragma unroll
    for (int hh = 0; hh < GP; ++hh)
#pragma unroll
      for (int e = 0; e < 8; ++e) s_acc[wave][hh][8 * c + e] = st.acc[hh][e];
  }
  if (lane == 0) {
#pragma unroll
    for (int hh = 0; hh < GP; ++hh) { s_m[wave][hh] = mh[hh]; s_l[wave][hh] = lh[hh]; }
  }
  __syncthreads();

  const int64_t part = (static_cast<int64_t>(b) * a.heads + h) * a.splits + split;
  for (int idx = threadIdx.x; idx < a.group * kHeadDim; idx += 64 * kWaves) {
    const int hh = idx / kHeadDim;
    const int d = idx % kHeadDim;
    float M = neg_inf();
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, s_m[w][hh]);
    const float Ms = (M == neg_inf()) ? 0.f : M;
    float L = 0.f, O = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = __builtin_amdgcn_exp2f(s_m[w][hh] - Ms);
      L += s_l[w][hh] * f;
      O += s_acc[w][hh][d] * f;
    }
    // L >= 1 whenever a token was seen (the maximum contributes exp2(0)), so
    // the hardware reciprocal and log2 need no denormal or zero handling.
    a.o_part[(part * a.group + hh) * kHeadDim + d] = L == 0.f ? 0.f : O * __builtin_amdgcn_rcpf(L);
    if (d == 0)
      a.lse_part[part * a.group + hh] = (L == 0.f) ? neg_inf() : (M + __builtin_amdgcn_logf(L)) * kLn2;
  }
}

// Combine: one 256-thread work-group per (sequence, kv head, query head,
// 32-dim quarter). Thread (sl, dq) folds splits sl, sl + 32, ... of dims
// 4*dq .. 4*dq+3 with a running (max, sum, weighted o); the 32 split lanes are
// merged with wave shuffles and one LDS exchange. All loads are issued before
// any is consumed, so a call costs one memory round trip.
constexpr int kCombineLanes = 32;   // split lanes per work-group
constexpr int kCombineQuads = 8;    // float4 dim quads per work-group (32 dims)

struct Acc4 {
  float m, l;
  float4 o;
};

__device__ __forceinline__ Acc4 merge(const Acc4& a, const Acc4& b) {
  const float M = fmaxf(a.m, b.m);
  const float Ms = (M == neg_inf()) ? 0.f : M;
  const float fa = __builtin_amdgcn_exp2f((a.m - Ms) * kLog2e);
  const float fb = __builtin_amdgcn_exp2f((b.m - Ms) * kLog2e);
  Acc4 r;
  r.m = M;
  r.l = a.l * fa + b.l * fb;
  r.o = make_float4(a.o.x * fa + b.o.x * fb, a.o.y * fa + b.o.y * fb, a.o.z * fa + b.o.z * fb,
                    a.o.w * fa + b.o.w * fb);
  return r;
}

__device__ __forceinline__ Acc4 shfl_xor(const Acc4& a, int mask) {
  Acc4 r;
  r.m = __shfl_xor(a.m, mask);
  r.l = __shfl_xor(a.l, mask);
  r.o = make_float4(__shfl_xor(a.o.x, mask), __shfl_xor(a.o.y, mask), __shfl_xor(a.o.z, mask),
                    __shfl_xor(a.o.w, mask));
  return r;
}

template <int DT>
__global__ __launch_bounds__(256) void decode_combine_kernel(const CombineArgs a) {
  using E = Elem<DT>;
  __shared__ Acc4 s_part[4][kCombineQuads];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int dq = tid & (kCombineQuads - 1);
  const int sl = tid / kCombineQuads;
  const int G = a.group;
  const int S = a.splits;
  const int64_t blk = blockIdx.x;
  const int quarter = static_cast<int>(blk & 3);
  const int64_t bhg = blk >> 2;
  const int g = static_cast<int>(bhg % G);
  const int64_t bh = bhg / G;
  const int h = static_cast<int>(bh % a.heads);
  const int64_t b = bh / a.heads;
  const int dim0 = 32 * quarter + 4 * dq;

  const float* lse = a.lse_part + bh * S * G + g;
  const float* o = a.o_part + (bh * S * G + g) * kHeadDim + dim0;

  Acc4 acc;
  acc.m = neg_inf();
  acc.l = 0.f;
  acc.o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 4
  for (int s = sl; s < S; s += kCombineLanes) {
    const float ls = lse[static_cast<int64_t>(s) * G];
    const float4 ov = *reinterpret_cast<const float4*>(o + static_cast<int64_t>(s) * G * kHeadDim);
    Acc4 one;
    one.m = ls;
    one.l = 1.f;
    one.o = ov;
    acc = merge(acc, one);
  }
  // Split lanes inside the wave: lanes dq + 8 * k, k = 0..7.
  acc = merge(acc, shfl_xor(acc, 8));
  acc = merge(acc, shfl_xor(acc, 16));
  acc = merge(acc, shfl_xor(acc, 32));
  if (lane < kCombineQuads) s_part[wave][lane] = acc;
  __syncthreads();
  if (tid < kCombineQuads) {
    Acc4 r = s_part[0][tid];
#pragma unroll
    for (int w = 1; w < 4; ++w) r = merge(r, s_part[w][tid]);
    const bool empty = (r.m == neg_inf());
    const float inv = empty ? 0.f : 1.f / r.l;
    const uint32_t w0 = E::bits(r.o.x * inv) | (E::bits(r.o.y * inv) << 16);
    const uint32_t w1 = E::bits(r.o.z * inv) | (E::bits(r.o.w * inv) << 16);
    uint16_t* dst = a.out + b * a.so_b + h * a.so_h + g * a.so_g + 32 * quarter + 4 * tid;
    *reinterpret_cast<uint2*>(dst) = make_uint2(w0, w1);
  }
}

// ---------------------------------------------------------------------------
// Host-side validation and launch.
// ---------------------------------------------------------------------------

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

template <int DT, int GP>
hipError_t launch_partial_t(const PartialArgs& a, int batch, hipStream_t stream) {
  hipLaunchKernelGGL((decode_partial_kernel<DT, GP>), dim3(a.splits, a.heads, batch), dim3(64 * kWaves), 0,
                     stream, a);
  return hipGetLastError();
}

template <int DT>
hipError_t launch_partial_dt(const PartialArgs& a, int batch, hipStream_t stream) {
  if (a.group <= 1) return launch_partial_t<DT, 1>(a, batch, stream);
  if (a.group <= 2) return launch_partial_t<DT, 2>(a, batch, stream);
  if (a.group <= 4) return launch_partial_t<DT, 4>(a, batch, stream);
  return launch_partial_t<DT, 8>(a, batch, stream);
}

// Split plan of a call: S splits of T tokens each (S * T >= n, T a multiple of
// the granule). With split_tokens > 0 the caller fixes T. Otherwise S is
// chosen so that B * Hkv * S work-groups are TC_DECODE_WGS_PER_CU per compute
// unit (every work-group then streams the same share of the cache when its
// tiles are dealt round-robin), but never more splits than a head has
// wave-tiles and never more than TC_MAX_SPLITS. Ragged batches (per-sequence
// lengths) aim at TC_DECODE_RAGGED_WGS_PER_CU per unit: short sequences leave
// their work-groups light, and many small work-groups let the dispatcher
// balance the rest.
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

int partial_impl(const void* q_dev, const int64_t q_strides[3], const void* k_dev, const int64_t k_strides[3],
                 const void* v_dev, const int64_t v_strides[3], const int32_t* lens_dev, int64_t n_tokens, int batch,
                 int kv_heads, int group, int head_dim, int dtype, float scale, int split_tokens, int num_splits,
                 float* o_part_dev, float* lse_part_dev, int interleave, const Append* app, void* stream) {
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
  a.k_new = app ? static_cast<const uint16_t*>(app->k_new) : nullptr;
  a.v_new = app ? static_cast<const uint16_t*>(app->v_new) : nullptr;
  a.skn_b = app ? app->kn_strides[0] : 0;
  a.skn_h = app ? app->kn_strides[1] : 0;
  a.svn_b = app ? app->vn_strides[0] : 0;
  a.svn_h = app ? app->vn_strides[1] : 0;
  a.k_w = app ? static_cast<uint16_t*>(app->k_cache) : nullptr;
  a.v_w = app ? static_cast<uint16_t*>(app->v_cache) : nullptr;
  a.scale_log2 = static_cast<float>(static_cast<double>(scale) * 1.4426950408889634);

  hipStream_t s = static_cast<hipStream_t>(stream);
  const hipError_t e = dtype == TC_DTYPE_F16 ? launch_partial_dt<TC_DTYPE_F16>(a, batch, s)
                                             : launch_partial_dt<TC_DTYPE_BF16>(a, batch, s);
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
  const int64_t blocks = static_cast<int64_t>(batch) * kv_heads * group * 4;
  if (blocks > 0x7fffffff) return fail(TC_ERR_INVALID_ARGUMENT, "too many (sequence, head) pairs");
  const dim3 grid(static_cast<unsigned>(blocks));
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == TC_DTYPE_F16)
    hipLaunchKernelGGL((decode_combine_kernel<TC_DTYPE_F16>), grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL((decode_combine_kernel<TC_DTYPE_BF16>), grid, dim3(256), 0, s, a);
  return hip_status(hipGetLastError(), "decode_combine launch");
}

}  // extern "C"

namespace tc {
namespace {

int attention_impl(const void* q_dev, const int64_t q_strides[3], const void* k_dev, const int64_t k_strides[3],
                   const void* v_dev, const int64_t v_strides[3], const int32_t* lens_dev, int64_t n_tokens,
                   int batch, int kv_heads, int group, int head_dim, int dtype, float scale, int split_tokens,
                   void* workspace_dev, size_t workspace_bytes, void* out_dev, const int64_t out_strides[3],
                   const Append* app, int ragged_plan, void* stream) {
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
                      head_dim, dtype, scale, t, S, o_part, lse_part, TC_DECODE_INTERLEAVE, app, stream);
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

}  // extern "C"
