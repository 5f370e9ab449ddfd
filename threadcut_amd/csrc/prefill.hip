// GQA-native prefill attention for gfx950 (MFMA, fp32 softmax).
//
// Reference semantics: the prefill branch of threadcut/attention.py:43-46 —
// SDPA of q [b, hq, L, d] against repeat_kv(k), repeat_kv(v) (each KV head
// expanded g = hq/hkv times) with the boolean attention mask, or is_causal
// when there is no mask and L == n; output transposed to [b, L, hq, d].
// Here the KV heads are never expanded: a work-group owns 64 query rows that
// are (query token, query head of the group) pairs of ONE KV head, so every
// K/V tile it stages in LDS is read from HBM once and shared by the g heads.
//
// Per 64-key tile, each wave (16 query rows) computes
//   S^T = K . Q^T   with v_mfma_f32_16x16x32_f16: A = K rows from LDS, B = Q^T
//                   from registers; lane l then holds keys 4(l/16)+r of query
//                   row l%16, so a row's softmax needs only 4 lanes;
//   O^T += V^T . P^T with P^T fed straight from those registers (fp16) and
//                   V^T from LDS (V is transposed while staged), so no
//                   cross-lane shuffle of P is needed.
// The online softmax (max, sum, rescale) runs per query row in fp32, log2
// domain. Tiles are double-buffered: the next tile's global loads are in
// flight while the current one is multiplied.
#include <cmath>

#include "tc_common.hpp"

namespace tc {
namespace {

constexpr int kHeadDim = 128;
constexpr int kRows = 64;          // query rows per work-group (4 waves x 16)
constexpr int kKeys = 64;          // keys per tile
constexpr int kKStride = 136;      // halfs per K row in LDS (256 B + 16 B pad)
constexpr int kVStride = 68;       // halfs per V^T row in LDS (128 B + 8 B pad)
constexpr int kKTile = kKeys * kKStride;
constexpr int kVTile = kHeadDim * kVStride;

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

struct PrefillArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  const uint8_t* mask;      // null, or [mb, L, n] booleans (batch stride 0 broadcasts)
  uint16_t* out;            // [b, L, hq, d]
  int64_t sq_b, sq_h, sq_t;
  int64_t sk_b, sk_h, sk_t;
  int64_t sv_b, sv_h, sv_t;
  int64_t sm_b, sm_q, sm_k;
  int64_t so_b, so_t, so_h;
  int64_t q_len, n;         // query tokens, keys (the queries sit at positions n - q_len ..)
  int kv_heads, causal;
  float scale_log2;
};

template <int DT> struct Mfma;
template <> struct Mfma<TC_DTYPE_F16> {
  static __device__ __forceinline__ float4v mma(const uint4& a, const uint4& b, float4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, a), __builtin_bit_cast(half8, b), c, 0,
                                                  0, 0);
  }
};
template <> struct Mfma<TC_DTYPE_BF16> {
  static __device__ __forceinline__ float4v mma(const uint4& a, const uint4& b, float4v c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0,
                                           static_cast<int32_t>(bytes < 0 ? 0 : (bytes > 0x7fffffff ? 0x7fffffff : bytes)),
                                           0x00020000);
}

__device__ __forceinline__ uint4 bload(__amdgpu_buffer_rsrc_t r, int32_t off) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Staged registers of one K/V tile: thread t holds K chunks (key c/16,
// dims 8*(c%16)) for c = t + 256*i, and V rows 4*(t/16)+i, dims 8*(t%16).
struct Stage {
  uint4 k[4];
  uint4 v[4];
};

__device__ __forceinline__ void load_stage(Stage& s, const char* kslab, const char* vslab, int64_t row_k,
                                           int64_t row_v, int64_t key0, int64_t n) {
  const int t = threadIdx.x;
  const int64_t rows = n - key0 < kKeys ? n - key0 : kKeys;
  const __amdgpu_buffer_rsrc_t rk = rsrc(kslab + key0 * row_k, rows * row_k);
  const __amdgpu_buffer_rsrc_t rv = rsrc(vslab + key0 * row_v, rows * row_v);
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = t + 256 * i;
    s.k[i] = bload(rk, static_cast<int32_t>((c >> 4) * row_k + 16 * (c & 15)));
    s.v[i] = bload(rv, static_cast<int32_t>((4 * (t >> 4) + i) * row_v + 16 * (t & 15)));
  }
}

// K rows as they are; V transposed to V^T[dim][key] (4 keys x 8 dims per thread).
__device__ __forceinline__ void store_stage(const Stage& s, uint16_t* lk, uint16_t* lv) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = t + 256 * i;
    *reinterpret_cast<uint4*>(lk + (c >> 4) * kKStride + 8 * (c & 15)) = s.k[i];
  }
  const int kq = t >> 4, dc = t & 15;
  const uint32_t* w0 = reinterpret_cast<const uint32_t*>(&s.v[0]);
  const uint32_t* w1 = reinterpret_cast<const uint32_t*>(&s.v[1]);
  const uint32_t* w2 = reinterpret_cast<const uint32_t*>(&s.v[2]);
  const uint32_t* w3 = reinterpret_cast<const uint32_t*>(&s.v[3]);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int sh = (e & 1) * 16;
    const uint32_t x0 = (w0[e >> 1] >> sh) & 0xffffu, x1 = (w1[e >> 1] >> sh) & 0xffffu;
    const uint32_t x2 = (w2[e >> 1] >> sh) & 0xffffu, x3 = (w3[e >> 1] >> sh) & 0xffffu;
    *reinterpret_cast<uint2*>(lv + (8 * dc + e) * kVStride + 4 * kq) = make_uint2(x0 | (x1 << 16), x2 | (x3 << 16));
  }
}

__device__ __forceinline__ float lanes4_max(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float lanes4_sum(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int DT, int G>
__global__ __launch_bounds__(256) void prefill_kernel(const PrefillArgs a) {
  using E = Elem<DT>;
  constexpr int kTokens = kRows / G;   // query tokens per work-group
  __shared__ uint16_t s_k[2][kKTile];
  __shared__ uint16_t s_v[2][kVTile];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int quad = lane >> 4;          // 0..3
  const int col = lane & 15;           // the lane's query row within the wave
  // Causal blocks run longest first (the last query block sees the most keys).
  const int64_t blk = a.causal ? static_cast<int64_t>(gridDim.x) - 1 - blockIdx.x : blockIdx.x;
  const int64_t tok0 = blk * kTokens;
  const int h = blockIdx.y;
  const int b = blockIdx.z;

  // This lane's query row: (token, head of the group).
  const int row = wave * 16 + col;
  const int64_t tok = tok0 + row / G;
  const int hq = h * G + row % G;
  const bool row_ok = tok < a.q_len;
  const int64_t past = a.n - a.q_len;
  const int64_t pos = past + tok;      // absolute position of the query token

  // Q^T as the MFMA B operand: dims 32c + 8*quad .. +8 of this lane's row.
  uint4 qb[4];
  {
    const uint16_t* qp = a.q + b * a.sq_b + hq * a.sq_h + (row_ok ? tok : 0) * a.sq_t + 8 * quad;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      qb[c] = row_ok ? *reinterpret_cast<const uint4*>(qp + 32 * c) : make_uint4(0u, 0u, 0u, 0u);
  }

  const char* kslab = reinterpret_cast<const char*>(a.k + b * a.sk_b + h * a.sk_h);
  const char* vslab = reinterpret_cast<const char*>(a.v + b * a.sv_b + h * a.sv_h);
  const int64_t row_k = a.sk_t * 2, row_v = a.sv_t * 2;
  const uint8_t* mrow = a.mask ? a.mask + b * a.sm_b + (row_ok ? tok : 0) * a.sm_q : nullptr;

  // Keys this work-group needs: all n, or up to its last query's position when causal.
  const int64_t last_tok = min(tok0 + kTokens, a.q_len) - 1;
  const int64_t key_end = a.causal ? min(a.n, past + last_tok + 1) : a.n;
  const int64_t ntiles = (key_end + kKeys - 1) / kKeys;

  float m = neg_inf(), l = 0.f;
  float4v o[8];
#pragma unroll
  for (int dt = 0; dt < 8; ++dt) o[dt] = float4v{0.f, 0.f, 0.f, 0.f};

  Stage st;
  if (ntiles > 0) {
    load_stage(st, kslab, vslab, row_k, row_v, 0, a.n);
    store_stage(st, s_k[0], s_v[0]);
  }
  __syncthreads();

  for (int64_t t = 0; t < ntiles; ++t) {
    const int buf = static_cast<int>(t & 1);
    const bool more = t + 1 < ntiles;
    if (more) load_stage(st, kslab, vslab, row_k, row_v, (t + 1) * kKeys, a.n);

    // S^T tile: 4 groups of 16 keys; lane holds keys 16*kt + 4*quad + r.
    const uint16_t* lk = s_k[buf];
    float4v s[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      float4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const uint4 ka = *reinterpret_cast<const uint4*>(lk + (16 * kt + col) * kKStride + 32 * c + 8 * quad);
        acc = Mfma<DT>::mma(ka, qb[c], acc);
      }
      s[kt] = acc;
    }

    // Scale, mask, running max of this row (4 lanes hold its 64 keys).
    const int64_t key0 = t * kKeys;
    float tmax = neg_inf();
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t key = key0 + 16 * kt + 4 * quad + r;
        bool ok = row_ok && key < a.n && (!a.causal || key <= pos);
        if (ok && mrow) ok = mrow[key * a.sm_k] != 0;
        const float x = ok ? s[kt][r] * a.scale_log2 : neg_inf();
        s[kt][r] = x;
        tmax = fmaxf(tmax, x);
      }
    tmax = lanes4_max(tmax);
    const float mn = fmaxf(m, tmax);
    const float ms = (mn == neg_inf()) ? 0.f : mn;
    const float alpha = __builtin_amdgcn_exp2f(m - ms);
    m = mn;

    // P^T as the B operand of two 32-key MFMA chunks: keys {4q..4q+3} of
    // group 2*kc and of group 2*kc+1, in that order (V^T is read to match).
    uint4 pb[2];
    float psum = 0.f;
#pragma unroll
    for (int kc = 0; kc < 2; ++kc) {
      uint32_t w[4];
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const float4v& x = s[2 * kc + half];
        const float p0 = __builtin_amdgcn_exp2f(x[0] - ms), p1 = __builtin_amdgcn_exp2f(x[1] - ms);
        const float p2 = __builtin_amdgcn_exp2f(x[2] - ms), p3 = __builtin_amdgcn_exp2f(x[3] - ms);
        psum += (p0 + p1) + (p2 + p3);
        w[2 * half] = E::bits(p0) | (E::bits(p1) << 16);
        w[2 * half + 1] = E::bits(p2) | (E::bits(p3) << 16);
      }
      pb[kc] = make_uint4(w[0], w[1], w[2], w[3]);
    }
    l = l * alpha + psum;

    const uint16_t* lv = s_v[buf];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      float4v acc = o[dt] * alpha;
#pragma unroll
      for (int kc = 0; kc < 2; ++kc) {
        const uint16_t* vp = lv + (16 * dt + col) * kVStride + 32 * kc + 4 * quad;
        const uint2 lo = *reinterpret_cast<const uint2*>(vp);
        const uint2 hi = *reinterpret_cast<const uint2*>(vp + 16);
        acc = Mfma<DT>::mma(make_uint4(lo.x, lo.y, hi.x, hi.y), pb[kc], acc);
      }
      o[dt] = acc;
    }

    if (more) store_stage(st, s_k[buf ^ 1], s_v[buf ^ 1]);
    __syncthreads();
  }

  // Normalize and write this lane's 32 outputs (dims 16*dt + 4*quad + r).
  const float lt = lanes4_sum(l);
  if (row_ok) {
    const float inv = lt > 0.f ? 1.f / lt : 0.f;
    uint16_t* op = a.out + b * a.so_b + tok * a.so_t + hq * a.so_h + 4 * quad;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      const uint32_t w0 = E::bits(o[dt][0] * inv) | (E::bits(o[dt][1] * inv) << 16);
      const uint32_t w1 = E::bits(o[dt][2] * inv) | (E::bits(o[dt][3] * inv) << 16);
      *reinterpret_cast<uint2*>(op + 16 * dt) = make_uint2(w0, w1);
    }
  }
}

template <int DT>
hipError_t launch_dt(const PrefillArgs& a, int group, int batch, hipStream_t stream) {
  const int tokens = kRows / group;
  const dim3 grid(static_cast<unsigned>((a.q_len + tokens - 1) / tokens), static_cast<unsigned>(a.kv_heads),
                  static_cast<unsigned>(batch));
  switch (group) {
    case 1: hipLaunchKernelGGL((prefill_kernel<DT, 1>), grid, dim3(256), 0, stream, a); break;
    case 2: hipLaunchKernelGGL((prefill_kernel<DT, 2>), grid, dim3(256), 0, stream, a); break;
    case 4: hipLaunchKernelGGL((prefill_kernel<DT, 4>), grid, dim3(256), 0, stream, a); break;
    default: hipLaunchKernelGGL((prefill_kernel<DT, 8>), grid, dim3(256), 0, stream, a); break;
  }
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

}  // namespace
}  // namespace tc

using namespace tc;

extern "C" int tc_prefill_attention(const void* q_dev, const int64_t q_strides[3], const void* k_dev,
                                    const int64_t k_strides[3], const void* v_dev, const int64_t v_strides[3],
                                    const uint8_t* mask_dev, const int64_t mask_strides[3], int causal,
                                    int64_t q_len, int64_t n_tokens, int batch, int q_heads, int kv_heads,
                                    int head_dim, int dtype, float scale, void* out_dev,
                                    const int64_t out_strides[3], void* stream) {
  clear_error();
  if (batch < 1 || batch > 65535 || kv_heads < 1 || kv_heads > 65535 || q_heads < 1)
    return fail(TC_ERR_INVALID_ARGUMENT, "batch %d, q_heads %d, kv_heads %d", batch, q_heads, kv_heads);
  if (q_heads % kv_heads) return fail(TC_ERR_INVALID_ARGUMENT, "q_heads %d not a multiple of kv_heads %d", q_heads, kv_heads);
  const int group = q_heads / kv_heads;
  if (group != 1 && group != 2 && group != 4 && group != 8)
    return fail(TC_ERR_UNSUPPORTED, "group %d unsupported (1, 2, 4 or 8)", group);
  if (head_dim != kHeadDim) return fail(TC_ERR_UNSUPPORTED, "head_dim %d unsupported (kernels are built for 128)", head_dim);
  if (dtype != TC_DTYPE_F16 && dtype != TC_DTYPE_BF16) return fail(TC_ERR_UNSUPPORTED, "dtype %d unsupported", dtype);
  if (q_len < 0 || n_tokens < q_len)
    return fail(TC_ERR_INVALID_ARGUMENT, "q_len %lld must be in [0, n_tokens %lld]", (long long)q_len,
                (long long)n_tokens);
  if (q_len == 0) return TC_OK;
  if (!q_dev || !k_dev || !v_dev || !out_dev) return fail(TC_ERR_INVALID_ARGUMENT, "null tensor pointer");
  if (!aligned16(q_dev) || !aligned16(k_dev) || !aligned16(v_dev) || !aligned16(out_dev))
    return fail(TC_ERR_ALIGNMENT, "q/k/v/out base pointers must be 16-byte aligned");
  int rc;
  if ((rc = check3("q", q_strides)) != TC_OK) return rc;
  if ((rc = check3("k", k_strides)) != TC_OK) return rc;
  if ((rc = check3("v", v_strides)) != TC_OK) return rc;
  if ((rc = check3("out", out_strides)) != TC_OK) return rc;
  // A 64-key tile is addressed with 32-bit buffer offsets: 64 rows of at most 2^24 elements.
  constexpr int64_t kMaxTokenStride = int64_t(1) << 24;
  if (k_strides[2] < head_dim || v_strides[2] < head_dim || k_strides[2] >= kMaxTokenStride ||
      v_strides[2] >= kMaxTokenStride)
    return fail(TC_ERR_INVALID_ARGUMENT, "k/v token strides outside [%d, 2^24)", head_dim);
  if (mask_dev && !mask_strides) return fail(TC_ERR_INVALID_ARGUMENT, "mask strides are null");
  if (mask_dev && causal) return fail(TC_ERR_INVALID_ARGUMENT, "pass either a mask or causal, not both");
  if (mask_dev && (mask_strides[0] < 0 || mask_strides[1] < 0 || mask_strides[2] < 0))
    return fail(TC_ERR_INVALID_ARGUMENT, "mask strides must be non-negative");
  if (!std::isfinite(scale)) return fail(TC_ERR_INVALID_ARGUMENT, "scale is not finite");

  PrefillArgs a;
  a.q = static_cast<const uint16_t*>(q_dev);
  a.k = static_cast<const uint16_t*>(k_dev);
  a.v = static_cast<const uint16_t*>(v_dev);
  a.mask = mask_dev;
  a.out = static_cast<uint16_t*>(out_dev);
  a.sq_b = q_strides[0]; a.sq_h = q_strides[1]; a.sq_t = q_strides[2];
  a.sk_b = k_strides[0]; a.sk_h = k_strides[1]; a.sk_t = k_strides[2];
  a.sv_b = v_strides[0]; a.sv_h = v_strides[1]; a.sv_t = v_strides[2];
  a.sm_b = mask_dev ? mask_strides[0] : 0;
  a.sm_q = mask_dev ? mask_strides[1] : 0;
  a.sm_k = mask_dev ? mask_strides[2] : 0;
  a.so_b = out_strides[0]; a.so_t = out_strides[1]; a.so_h = out_strides[2];
  a.q_len = q_len;
  a.n = n_tokens;
  a.kv_heads = kv_heads;
  a.causal = causal ? 1 : 0;
  a.scale_log2 = static_cast<float>(static_cast<double>(scale) * 1.4426950408889634);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const hipError_t e = dtype == TC_DTYPE_F16 ? launch_dt<TC_DTYPE_F16>(a, group, batch, s)
                                             : launch_dt<TC_DTYPE_BF16>(a, group, batch, s);
  return hip_status(e, "prefill launch");
}
