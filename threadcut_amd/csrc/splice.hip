// RoPE delta-shift of post-RoPE keys and the suffix splice of a KV cache.
//
// Reference semantics: threadcut/kv.py:15-25 (rotate_half and shift_keys:
// fp32 math, out = k*cos(emb) + rotate_half(k)*sin(emb), cast back) and
// :28-41, :83-92 (splice: K[a:a+c] <- shift(K[c0:c0+c], -gap), V[a:a+c] <-
// V[c0:c0+c], read before written; index_select variant for plain layers).
//
// One launch moves every (layer, K|V, batch row, head) strip of the cache.
// A thread owns one 16-byte chunk of the lower half of a row (dims 8u..8u+7)
// and the matching chunk of the upper half (64+8u..), which is exactly the
// pair rotate_half mixes, so each K row is gathered, rotated in fp32 and
// stored with no intermediate buffer; V rows take the same path unrotated.
// 8 threads cover a row, a pass of 256 threads covers 32 rows, and a thread
// keeps kUnroll passes of loads in flight before it stores.
#include <algorithm>

#include "tc_common.hpp"

namespace tc {
namespace {

constexpr int kHeadDim = 128;
constexpr int kHalf = kHeadDim / 2;
constexpr int kThreads = 256;
constexpr int kRowsPerPass = kThreads / 8;
#ifndef TC_SPLICE_UNROLL
#define TC_SPLICE_UNROLL 1  // passes of loads a thread keeps in flight (1 measured best: most work-groups)
#endif
#ifndef TC_SPLICE_NT
#define TC_SPLICE_NT 1      // non-temporal loads and stores (the strips are touched once)
#endif
constexpr int kUnroll = TC_SPLICE_UNROLL;
constexpr int kTileRows = kRowsPerPass * kUnroll;  // rows per work-group tile
constexpr int kMaxJobs = 128;                      // strips sets per launch (64 layers x K,V)
#ifndef TC_SPLICE_CHAIN_MIN
#define TC_SPLICE_CHAIN_MIN 46
#endif
// An overlapping move (gap < rows moved) with a gap of at least this many rows
// runs as gap independent chains per strip, one thread walking each
// (splice_kernel with DEPTH > 0); shorter gaps walk each strip in row order
// with one work-group. Chains win once the second work-group per strip has
// most of its 32 chains: 36 layers x 12188 rows, gap 47 753-760 us chained
// against 757-783 us walked, gap 44 757-779 either way, gaps 33-43 walked
// 6-60 us faster.
constexpr int64_t kChainMin = TC_SPLICE_CHAIN_MIN;
// An overlapping move with a shorter gap walks each strip in row order, cut
// into up to this many segments of at least kWalkMinRows rows that one
// work-group walks together (splice_walk_kernel). 36 layers x 12188 rows:
// two segments 727-769 us across gaps 1-47, against 760-780 us for one walk
// per strip; three, four and eight segments, or two rows per thread and
// pass, are slower (more concurrent streams or bytes in flight cost more than
// they hide).
#ifndef TC_SPLICE_WALK_SEGMENTS
#define TC_SPLICE_WALK_SEGMENTS 2
#endif
#ifndef TC_SPLICE_WALK_MIN_ROWS
#define TC_SPLICE_WALK_MIN_ROWS 256
#endif
constexpr int kWalkSegments = TC_SPLICE_WALK_SEGMENTS;
constexpr int64_t kWalkMinRows = TC_SPLICE_WALK_MIN_ROWS;
static_assert(kWalkSegments == 1 || kWalkSegments == 2 || kWalkSegments == 4 || kWalkSegments == 8,
              "walk segments: 1, 2, 4 or 8");
// Chain rows a thread loads before it stores them: 8 holds a whole chain of up
// to 8 rows at 128 VGPRs; longer chains run faster with 16 (235 VGPRs) in
// flight, shorter ones slower (occupancy). For long chains 8 or 6 rows (three
// or four waves per SIMD) measured 2-5% slower than 16 at gaps 47-1000.
constexpr int kChainDepthShort = 8;
constexpr int kChainDepthLong = 16;
// Dynamic LDS the row kernel is launched with and never touches: 26 KB of a
// CU's 160 KB holds residency at 6 work-groups (24 waves) per CU instead of 8.
// The parallel move of 36 layers x 5668 rows takes 282 us so against 290 us
// at 8 per CU; 4 per CU measured the same as 8, 5 and 7 between, 3 and 2
// far slower.
constexpr unsigned kRowKernelLds = 26624;

struct SpliceArgs {
  const uint16_t* src[kMaxJobs];
  uint16_t* dst[kMaxJobs];
  float cs[kHeadDim];  // cos(angle_i) for i < 64, then sin(angle_i)
  int64_t ss_b, ss_h, ss_t;
  int64_t ds_b, ds_h, ds_t;
  int64_t src_row0, dst_row0, rows;
  int heads;
  int rot_jobs;    // jobs [0, rot_jobs) are keys (rotated), the rest copied
  int64_t chain;   // > 0: chain walk of a move whose gap (src_row0 - dst_row0) is chain
  // Row walk (splice_walk_kernel): segments of seg_rows rows (a multiple of
  // the pass), the last one shorter; gap = src_row0 - dst_row0 < rows.
  int segments;
  int64_t seg_rows;
};

__device__ __forceinline__ uint4 load16(const uint16_t* p) {
#if TC_SPLICE_NT
  typedef unsigned int v4u __attribute__((ext_vector_type(4)));
  const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
#else
  return *reinterpret_cast<const uint4*>(p);
#endif
}

__device__ __forceinline__ void store16(uint16_t* p, const uint4& x) {
#if TC_SPLICE_NT
  typedef unsigned int v4u __attribute__((ext_vector_type(4)));
  v4u v = {x.x, x.y, x.z, x.w};
  __builtin_nontemporal_store(v, reinterpret_cast<v4u*>(p));
#else
  *reinterpret_cast<uint4*>(p) = x;
#endif
}

// out = fp(fl(x*cos) + fl(rotate_half(x)*sin)) per element, no contraction:
// lower half  y = x_lo*cos - x_hi*sin,  upper half y = x_hi*cos + x_lo*sin.
template <int DT>
__device__ __forceinline__ void rotate_pair(uint4& lo, uint4& hi, const float (&cv)[8], const float (&sv)[8]) {
#pragma clang fp contract(off)
  using E = Elem<DT>;
  uint32_t wl[4] = {lo.x, lo.y, lo.z, lo.w};
  uint32_t wh[4] = {hi.x, hi.y, hi.z, hi.w};
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const float c0 = cv[2 * w], c1 = cv[2 * w + 1];
    const float s0 = sv[2 * w], s1 = sv[2 * w + 1];
    const float xl0 = E::lo(wl[w]), xl1 = E::hi(wl[w]);
    const float xh0 = E::lo(wh[w]), xh1 = E::hi(wh[w]);
    const float yl0 = xl0 * c0 - xh0 * s0;
    const float yl1 = xl1 * c1 - xh1 * s1;
    const float yh0 = xh0 * c0 + xl0 * s0;
    const float yh1 = xh1 * c1 + xl1 * s1;
    wl[w] = E::bits(yl0) | (E::bits(yl1) << 16);
    wh[w] = E::bits(yh0) | (E::bits(yh1) << 16);
  }
  lo = make_uint4(wl[0], wl[1], wl[2], wl[3]);
  hi = make_uint4(wh[0], wh[1], wh[2], wh[3]);
}

template <int DT, int DEPTH>
__global__ __launch_bounds__(kThreads) void splice_kernel(const SpliceArgs a) {
  const int job = blockIdx.z;
  const int64_t bh = blockIdx.y;
  const int64_t b = bh / a.heads;
  const int64_t h = bh % a.heads;
  const bool rot = job < a.rot_jobs;
  const int r_in = threadIdx.x >> 3;  // row inside a pass
  const int u = threadIdx.x & 7;      // 16-byte chunk of each half row

  const uint16_t* src = a.src[job] + b * a.ss_b + h * a.ss_h + 8 * u;
  uint16_t* dst = a.dst[job] + b * a.ds_b + h * a.ds_h + 8 * u;

  // cos/sin of the thread's 8 frequency pairs (dims 8u..8u+7 and 64+8u..).
  float cv[8], sv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    cv[i] = a.cs[8 * u + i];
    sv[i] = a.cs[kHalf + 8 * u + i];
  }

  if constexpr (DEPTH > 0) {
    // Chain walk. Destination row r takes source row r + gap, so the rows
    // j, j + gap, j + 2 gap ... (j < gap) form a chain that reads and writes
    // only its own rows: each row is read as the source of the chain's
    // previous row and then overwritten by the next one's. A thread walks one
    // chain's 16-byte chunks in order. The store to row r overwrites what the
    // same thread loaded for row r - gap, whose value an earlier store of this
    // thread has already consumed, so no other thread and no barrier is involved.
    const int64_t j = static_cast<int64_t>(blockIdx.x) * kRowsPerPass + r_in;
    if (j >= a.chain) return;
    for (int64_t r0 = j; r0 < a.rows; r0 += DEPTH * a.chain) {
      uint4 lo[DEPTH], hi[DEPTH];
#pragma unroll
      for (int i = 0; i < DEPTH; ++i) {
        const int64_t r = r0 + i * a.chain;
        if (r < a.rows) {
          const uint16_t* p = src + (a.src_row0 + r) * a.ss_t;
          lo[i] = load16(p);
          hi[i] = load16(p + kHalf);
        }
      }
#pragma unroll
      for (int i = 0; i < DEPTH; ++i) {
        const int64_t r = r0 + i * a.chain;
        if (r < a.rows) {
          if (rot) rotate_pair<DT>(lo[i], hi[i], cv, sv);
          uint16_t* p = dst + (a.dst_row0 + r) * a.ds_t;
          store16(p, lo[i]);
          store16(p + kHalf, hi[i]);
        }
      }
    }
    return;
  }

  int64_t row = static_cast<int64_t>(blockIdx.x) * kTileRows;
  const int64_t row_end = min(row + kTileRows, a.rows);
  for (; row < row_end; row += kTileRows) {
    uint4 lo[kUnroll], hi[kUnroll];
#pragma unroll
    for (int i = 0; i < kUnroll; ++i) {
      const int64_t r = row + i * kRowsPerPass + r_in;
      if (r < row_end) {
        const uint16_t* p = src + (a.src_row0 + r) * a.ss_t;
        lo[i] = load16(p);
        hi[i] = load16(p + kHalf);
      }
    }
#pragma unroll
    for (int i = 0; i < kUnroll; ++i) {
      const int64_t r = row + i * kRowsPerPass + r_in;
      if (r < row_end) {
        if (rot) rotate_pair<DT>(lo[i], hi[i], cv, sv);
        uint16_t* p = dst + (a.dst_row0 + r) * a.ds_t;
        store16(p, lo[i]);
        store16(p + kHalf, hi[i]);
      }
    }
  }
}

// Overlapping move with a short gap, one work-group per strip. Destination
// row r takes source row r + gap. The strip's rows are cut into segments of
// seg_rows rows, walked together in row order, one 32-row pass of every
// segment at a time: every load of a pass lands before any store of it (a
// pass's sources reach gap rows into its own destinations), and the next
// pass's sources lie past this pass's destinations. A segment's last gap
// source rows are the next segment's first gap destination rows, which that
// segment overwrites in its first pass: they are copied to LDS (the halo)
// before any store and read from there.
template <int DT, int SEG>
__global__ __launch_bounds__(kThreads) void splice_walk_kernel(const SpliceArgs a) {
  extern __shared__ uint4 halo[];  // [(segments - 1) * gap rows][16 chunks]
  const int job = blockIdx.z;
  const int64_t bh = blockIdx.y;
  const int64_t b = bh / a.heads;
  const int64_t h = bh % a.heads;
  const bool rot = job < a.rot_jobs;
  const int r_in = threadIdx.x >> 3;
  const int u = threadIdx.x & 7;
  const int64_t gap = a.src_row0 - a.dst_row0;
  const int64_t L = a.seg_rows;
  const int segs = a.segments;

  const uint16_t* src_strip = a.src[job] + b * a.ss_b + h * a.ss_h;
  const uint16_t* src = src_strip + 8 * u;
  uint16_t* dst = a.dst[job] + b * a.ds_b + h * a.ds_h + 8 * u;

  float cv[8], sv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    cv[i] = a.cs[8 * u + i];
    sv[i] = a.cs[kHalf + 8 * u + i];
  }

  // Halo k, row j: source row (k + 1) L - gap + j of segment k.
  const int64_t halo_chunks = (segs - 1) * gap * 8;
  for (int64_t i = threadIdx.x; i < halo_chunks; i += kThreads) {
    const int64_t k = i / (gap * 8);
    const int64_t j = (i >> 3) - k * gap;
    const int uu = static_cast<int>(i & 7);
    const uint16_t* p = src_strip + (a.src_row0 + (k + 1) * L - gap + j) * a.ss_t + 8 * uu;
    halo[(k * gap + j) * 16 + uu] = load16(p);
    halo[(k * gap + j) * 16 + 8 + uu] = load16(p + kHalf);
  }
  __syncthreads();

  for (int64_t off = 0; off < L; off += kRowsPerPass) {
    uint4 lo[SEG], hi[SEG];
#pragma unroll
    for (int k = 0; k < SEG; ++k) {
      const int64_t r = k * L + off + r_in;
      if (k < segs && r < min((k + 1) * L, a.rows)) {
        const int64_t j = r - ((k + 1) * L - gap);
        if (k < segs - 1 && j >= 0) {
          lo[k] = halo[(k * gap + j) * 16 + u];
          hi[k] = halo[(k * gap + j) * 16 + 8 + u];
        } else {
          const uint16_t* p = src + (a.src_row0 + r) * a.ss_t;
          lo[k] = load16(p);
          hi[k] = load16(p + kHalf);
        }
      }
    }
    __asm__ volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
#pragma unroll
    for (int k = 0; k < SEG; ++k) {
      const int64_t r = k * L + off + r_in;
      if (k < segs && r < min((k + 1) * L, a.rows)) {
        if (rot) rotate_pair<DT>(lo[k], hi[k], cv, sv);
        uint16_t* p = dst + (a.dst_row0 + r) * a.ds_t;
        store16(p, lo[k]);
        store16(p + kHalf, hi[k]);
      }
    }
  }
}

// Paged cache prune: the kept suffix's keys re-rotated in place in their
// pages. Each tile entry is {page, first slot, rows (<= 16), 0}, the format
// of the paged decode's tile table; entries outside the pool or past a page's
// end are skipped. A work-group covers two tiles of one (layer, head): thread
// (tile half, row, 16-byte chunk u), which loads, rotates and stores its own
// chunks, so the in-place update needs no ordering between threads.
struct PagedRotateArgs {
  uint16_t* k[kMaxJobs];  // the layers' K pools
  float cs[kHeadDim];     // cos(angle_i) for i < 64, then sin(angle_i)
  int64_t sp, sh, st;     // pool strides: page, head, token
  const int32_t* tiles;   // [num_tiles, 4]
  int64_t num_tiles;
  int pages, page_tokens;
};

template <int DT>
__global__ __launch_bounds__(kThreads) void paged_rotate_kernel(const PagedRotateArgs a) {
  const int64_t tile = 2 * static_cast<int64_t>(blockIdx.x) + (threadIdx.x >> 7);
  const int row = (threadIdx.x >> 3) & 15;
  const int u = threadIdx.x & 7;
  if (tile >= a.num_tiles) return;
  const int4 e = *reinterpret_cast<const int4*>(a.tiles + 4 * tile);
  if (e.x < 0 || e.x >= a.pages || e.y < 0 || e.z < 0 || e.z > 16 || e.y > a.page_tokens - e.z) return;
  if (row >= e.z) return;
  float cv[8], sv[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    cv[i] = a.cs[8 * u + i];
    sv[i] = a.cs[kHalf + 8 * u + i];
  }
  uint16_t* p = a.k[blockIdx.z] + e.x * a.sp + static_cast<int64_t>(blockIdx.y) * a.sh + (e.y + row) * a.st + 8 * u;
  uint4 lo = load16(p), hi = load16(p + kHalf);
  rotate_pair<DT>(lo, hi, cv, sv);
  store16(p, lo);
  store16(p + kHalf, hi);
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------

int check_dims(int batch, int heads, int head_dim, int dtype) {
  if (batch < 1 || heads < 1 || static_cast<int64_t>(batch) * heads > 65535)
    return fail(TC_ERR_INVALID_ARGUMENT, "batch %d x heads %d outside [1, 65535]", batch, heads);
  if (head_dim != kHeadDim) return fail(TC_ERR_UNSUPPORTED, "head_dim %d unsupported (kernels are built for 128)", head_dim);
  if (dtype != TC_DTYPE_F16 && dtype != TC_DTYPE_BF16) return fail(TC_ERR_UNSUPPORTED, "dtype %d unsupported", dtype);
  return TC_OK;
}

int check_strides3(const char* what, const int64_t* st) {
  if (!st) return fail(TC_ERR_INVALID_ARGUMENT, "%s strides are null", what);
  for (int i = 0; i < 3; ++i) {
    if (st[i] < 0) return fail(TC_ERR_INVALID_ARGUMENT, "%s stride %d is negative", what, i);
    if (st[i] % 8) return fail(TC_ERR_ALIGNMENT, "%s stride %d (%lld) not a multiple of 8", what, i, (long long)st[i]);
  }
  if (st[2] < kHeadDim) return fail(TC_ERR_INVALID_ARGUMENT, "%s token stride %lld overlaps rows", what, (long long)st[2]);
  return TC_OK;
}

int check_ptrs(const char* what, void* const* ptrs, int n) {
  if (n > 0 && !ptrs) return fail(TC_ERR_INVALID_ARGUMENT, "%s pointer array is null", what);
  for (int i = 0; i < n; ++i) {
    if (!ptrs[i]) return fail(TC_ERR_INVALID_ARGUMENT, "%s[%d] is null", what, i);
    if (!aligned16(ptrs[i])) return fail(TC_ERR_ALIGNMENT, "%s[%d] is not 16-byte aligned", what, i);
  }
  return TC_OK;
}

template <int SEG>
void launch_walk(bool f16, dim3 grid, unsigned lds, hipStream_t stream, const SpliceArgs& a) {
  if (f16)
    hipLaunchKernelGGL((splice_walk_kernel<TC_DTYPE_F16, SEG>), grid, dim3(kThreads), lds, stream, a);
  else
    hipLaunchKernelGGL((splice_walk_kernel<TC_DTYPE_BF16, SEG>), grid, dim3(kThreads), lds, stream, a);
}

template <int DEPTH>
void launch_kernel(bool f16, dim3 grid, hipStream_t stream, const SpliceArgs& a) {
  const unsigned lds = DEPTH > 0 ? 0 : kRowKernelLds;
  if (f16)
    hipLaunchKernelGGL((splice_kernel<TC_DTYPE_F16, DEPTH>), grid, dim3(kThreads), lds, stream, a);
  else
    hipLaunchKernelGGL((splice_kernel<TC_DTYPE_BF16, DEPTH>), grid, dim3(kThreads), lds, stream, a);
}

// Launches the kernel over `layers` layers, K strips rotated when `rotate`;
// vsrc == nullptr moves keys only.
int launch_rows(void* const* ksrc, void* const* vsrc, void* const* kdst, void* const* vdst, int layers,
                const int64_t* ss, const int64_t* ds, int batch, int heads, int dtype, int64_t src_row0,
                int64_t dst_row0, int64_t rows, bool rotate, bool sequential, const float* cos_sin,
                hipStream_t stream, int64_t chain = 0) {
  if (rows <= 0 || layers <= 0) return TC_OK;
  constexpr int kLayersPerLaunch = kMaxJobs / 2;
  const int per_layer = vsrc ? 2 : 1;
  for (int l0 = 0; l0 < layers; l0 += kLayersPerLaunch) {
    const int nl = min(kLayersPerLaunch, layers - l0);
    SpliceArgs a;
    for (int i = 0; i < nl; ++i) {
      a.src[i] = static_cast<const uint16_t*>(ksrc[l0 + i]);
      a.dst[i] = static_cast<uint16_t*>(kdst[l0 + i]);
      if (vsrc) {
        a.src[nl + i] = static_cast<const uint16_t*>(vsrc[l0 + i]);
        a.dst[nl + i] = static_cast<uint16_t*>(vdst[l0 + i]);
      }
    }
    for (int i = per_layer * nl; i < kMaxJobs; ++i) { a.src[i] = nullptr; a.dst[i] = nullptr; }
    for (int i = 0; i < kHeadDim; ++i) a.cs[i] = (rotate && cos_sin) ? cos_sin[i] : 0.f;
    a.ss_b = ss[0]; a.ss_h = ss[1]; a.ss_t = ss[2];
    a.ds_b = ds[0]; a.ds_h = ds[1]; a.ds_t = ds[2];
    a.src_row0 = src_row0;
    a.dst_row0 = dst_row0;
    a.rows = rows;
    a.heads = heads;
    a.rot_jobs = rotate ? nl : 0;
    a.chain = chain;
    a.segments = 1;
    a.seg_rows = rows;
    const int64_t tiles = chain > 0 ? ceil_div(min(chain, rows), kRowsPerPass)
                                    : sequential ? 1 : ceil_div(rows, kTileRows);
    if (tiles > 0x7fffffff) return fail(TC_ERR_INVALID_ARGUMENT, "too many rows (%lld)", (long long)rows);
    const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(batch * heads),
                    static_cast<unsigned>(per_layer * nl));
    const int depth = chain <= 0 ? 0 : rows > kChainDepthShort * chain ? kChainDepthLong : kChainDepthShort;
    const bool f16 = dtype == TC_DTYPE_F16;
    if (sequential) {
      // Segments of at least kWalkMinRows rows (and at least the gap, so a
      // halo lies in its own segment's sources), a whole number of passes.
      const int64_t gap = src_row0 - dst_row0;
      if (gap <= 0 || gap >= rows || gap >= kChainMin)
        return fail(TC_ERR_INVALID_ARGUMENT, "row walk of gap %lld over %lld rows", (long long)gap, (long long)rows);
      const int64_t want = std::max<int64_t>(1, std::min<int64_t>(kWalkSegments, ceil_div(rows, kWalkMinRows)));
      int64_t L = ceil_div(ceil_div(rows, want), kRowsPerPass) * kRowsPerPass;
      L = std::max(L, ceil_div(gap, kRowsPerPass) * kRowsPerPass);
      a.seg_rows = L;
      a.segments = static_cast<int>(ceil_div(rows, L));
      const unsigned lds = static_cast<unsigned>((a.segments - 1) * gap * kHeadDim * 2);
      if (a.segments <= 1)
        launch_walk<1>(f16, grid, lds, stream, a);
      else
        launch_walk<kWalkSegments>(f16, grid, lds, stream, a);
    } else if (depth == kChainDepthLong)
      launch_kernel<kChainDepthLong>(f16, grid, stream, a);
    else if (depth == kChainDepthShort)
      launch_kernel<kChainDepthShort>(f16, grid, stream, a);
    else
      launch_kernel<0>(f16, grid, stream, a);
    const int rc = hip_status(hipGetLastError(), "splice launch");
    if (rc != TC_OK) return rc;
  }
  return TC_OK;
}

}  // namespace
}  // namespace tc

using namespace tc;

extern "C" {

int tc_shift_keys(const void* keys_dev, const int64_t src_strides[3], void* out_dev, const int64_t dst_strides[3],
                  int batch, int heads, int64_t tokens, int head_dim, int dtype, const float* cos_sin_host,
                  void* stream) {
  clear_error();
  int rc = check_dims(batch, heads, head_dim, dtype);
  if (rc != TC_OK) return rc;
  if ((rc = check_strides3("keys", src_strides)) != TC_OK) return rc;
  if ((rc = check_strides3("out", dst_strides)) != TC_OK) return rc;
  if (tokens < 0) return fail(TC_ERR_INVALID_ARGUMENT, "tokens %lld is negative", (long long)tokens);
  if (tokens == 0) return TC_OK;
  if (!keys_dev || !out_dev || !cos_sin_host) return fail(TC_ERR_INVALID_ARGUMENT, "null pointer");
  if (!aligned16(keys_dev) || !aligned16(out_dev)) return fail(TC_ERR_ALIGNMENT, "keys/out not 16-byte aligned");
  if (keys_dev == out_dev) return fail(TC_ERR_INVALID_ARGUMENT, "out may not alias keys");
  void* k = const_cast<void*>(keys_dev);
  void* o = out_dev;
  return launch_rows(&k, nullptr, &o, nullptr, 1, src_strides, dst_strides, batch, heads, dtype, 0, 0, tokens, true,
                     false, cos_sin_host, static_cast<hipStream_t>(stream));
}

int tc_splice_rope(void* const* k_layers_host, void* const* v_layers_host, int num_layers, const int64_t strides[3],
                   int batch, int heads, int64_t capacity, int head_dim, int dtype, int64_t a, int64_t c0, int64_t c,
                   const float* cos_sin_host, void* stream) {
  clear_error();
  int rc = check_dims(batch, heads, head_dim, dtype);
  if (rc != TC_OK) return rc;
  if (num_layers < 0) return fail(TC_ERR_INVALID_ARGUMENT, "num_layers %d is negative", num_layers);
  if ((rc = check_strides3("cache", strides)) != TC_OK) return rc;
  if (a < 0 || c < 0 || c0 < a)
    return fail(TC_ERR_INVALID_ARGUMENT, "split (a=%lld, c0=%lld, c=%lld) needs 0 <= a <= c0 and c >= 0", (long long)a,
                (long long)c0, (long long)c);
  if (c0 + c > capacity)
    return fail(TC_ERR_INVALID_ARGUMENT, "suffix [%lld, %lld) past the capacity %lld", (long long)c0,
                (long long)(c0 + c), (long long)capacity);
  if ((rc = check_ptrs("k_layers", k_layers_host, num_layers)) != TC_OK) return rc;
  if ((rc = check_ptrs("v_layers", v_layers_host, num_layers)) != TC_OK) return rc;
  if (c == 0 || c0 == a || num_layers == 0) return TC_OK;
  if (!cos_sin_host) return fail(TC_ERR_INVALID_ARGUMENT, "cos_sin table is null");
  const int64_t gap = c0 - a;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (gap >= c)  // disjoint ranges: every row in parallel
    return launch_rows(k_layers_host, v_layers_host, k_layers_host, v_layers_host, num_layers, strides, strides,
                       batch, heads, dtype, c0, a, c, true, false, cos_sin_host, s);
  if (gap < kChainMin)  // overlapping, short gap: one work-group walks each strip in row order, in segments
    return launch_rows(k_layers_host, v_layers_host, k_layers_host, v_layers_host, num_layers, strides, strides,
                       batch, heads, dtype, c0, a, c, true, true, cos_sin_host, s);
  // Overlapping: gap independent chains per strip.
  return launch_rows(k_layers_host, v_layers_host, k_layers_host, v_layers_host, num_layers, strides, strides,
                     batch, heads, dtype, c0, a, c, true, false, cos_sin_host, s, gap);
}

int tc_splice_copy(void* const* k_src_host, void* const* v_src_host, const int64_t src_strides[3], int64_t src_tokens,
                   void* const* k_dst_host, void* const* v_dst_host, const int64_t dst_strides[3], int num_layers,
                   int batch, int heads, int head_dim, int dtype, int64_t a, int64_t c0, int64_t c,
                   const float* cos_sin_host, void* stream) {
  clear_error();
  int rc = check_dims(batch, heads, head_dim, dtype);
  if (rc != TC_OK) return rc;
  if (num_layers < 0) return fail(TC_ERR_INVALID_ARGUMENT, "num_layers %d is negative", num_layers);
  if ((rc = check_strides3("src", src_strides)) != TC_OK) return rc;
  if ((rc = check_strides3("dst", dst_strides)) != TC_OK) return rc;
  if (a < 0 || c < 0 || c0 < a)
    return fail(TC_ERR_INVALID_ARGUMENT, "split (a=%lld, c0=%lld, c=%lld) needs 0 <= a <= c0 and c >= 0", (long long)a,
                (long long)c0, (long long)c);
  if (c0 + c > src_tokens || a > src_tokens)
    return fail(TC_ERR_INVALID_ARGUMENT, "split past the %lld source tokens", (long long)src_tokens);
  if (a + c == 0) return TC_OK;  // nothing kept: the destination is empty and needs no pointers
  if ((rc = check_ptrs("k_src", k_src_host, num_layers)) != TC_OK) return rc;
  if ((rc = check_ptrs("v_src", v_src_host, num_layers)) != TC_OK) return rc;
  if ((rc = check_ptrs("k_dst", k_dst_host, num_layers)) != TC_OK) return rc;
  if ((rc = check_ptrs("v_dst", v_dst_host, num_layers)) != TC_OK) return rc;
  const bool rotate = c > 0 && c0 != a;
  if (rotate && !cos_sin_host) return fail(TC_ERR_INVALID_ARGUMENT, "cos_sin table is null");
  hipStream_t s = static_cast<hipStream_t>(stream);
  rc = launch_rows(k_src_host, v_src_host, k_dst_host, v_dst_host, num_layers, src_strides, dst_strides, batch, heads,
                   dtype, 0, 0, a, false, false, nullptr, s);
  if (rc != TC_OK) return rc;
  return launch_rows(k_src_host, v_src_host, k_dst_host, v_dst_host, num_layers, src_strides, dst_strides, batch,
                     heads, dtype, c0, a, c, rotate, false, cos_sin_host, s);
}

int tc_paged_rotate_keys(void* const* k_pools_host, int num_layers, const int64_t pool_strides[3], int num_pages,
                         int page_tokens, const int32_t* tiles_dev, int64_t num_tiles, int kv_heads, int head_dim,
                         int dtype, const float* cos_sin_host, void* stream) {
  clear_error();
  int rc = check_dims(1, kv_heads, head_dim, dtype);
  if (rc != TC_OK) return rc;
  if (num_layers < 0) return fail(TC_ERR_INVALID_ARGUMENT, "num_layers %d is negative", num_layers);
  if (num_pages < 1 || page_tokens < 1)
    return fail(TC_ERR_INVALID_ARGUMENT, "pool of %d pages of %d tokens", num_pages, page_tokens);
  if ((rc = check_strides3("pool", pool_strides)) != TC_OK) return rc;
  if (num_tiles < 0) return fail(TC_ERR_INVALID_ARGUMENT, "num_tiles %lld is negative", (long long)num_tiles);
  if ((rc = check_ptrs("k_pools", k_pools_host, num_layers)) != TC_OK) return rc;
  if (num_tiles == 0 || num_layers == 0) return TC_OK;
  if (!tiles_dev) return fail(TC_ERR_INVALID_ARGUMENT, "null tile list");
  if (!aligned16(tiles_dev)) return fail(TC_ERR_ALIGNMENT, "tile list not 16-byte aligned");
  if (!cos_sin_host) return fail(TC_ERR_INVALID_ARGUMENT, "cos_sin table is null");
  const int64_t groups = ceil_div(num_tiles, 2);
  if (groups > 0x7fffffff) return fail(TC_ERR_INVALID_ARGUMENT, "too many tiles (%lld)", (long long)num_tiles);
  hipStream_t s = static_cast<hipStream_t>(stream);
  for (int l0 = 0; l0 < num_layers; l0 += kMaxJobs) {
    const int nl = min(kMaxJobs, num_layers - l0);
    PagedRotateArgs a;
    for (int i = 0; i < kMaxJobs; ++i) a.k[i] = i < nl ? static_cast<uint16_t*>(k_pools_host[l0 + i]) : nullptr;
    for (int i = 0; i < kHeadDim; ++i) a.cs[i] = cos_sin_host[i];
    a.sp = pool_strides[0]; a.sh = pool_strides[1]; a.st = pool_strides[2];
    a.tiles = tiles_dev;
    a.num_tiles = num_tiles;
    a.pages = num_pages;
    a.page_tokens = page_tokens;
    const dim3 grid(static_cast<unsigned>(groups), static_cast<unsigned>(kv_heads), static_cast<unsigned>(nl));
    if (dtype == TC_DTYPE_F16)
      hipLaunchKernelGGL((paged_rotate_kernel<TC_DTYPE_F16>), grid, dim3(kThreads), 0, s, a);
    else
      hipLaunchKernelGGL((paged_rotate_kernel<TC_DTYPE_BF16>), grid, dim3(kThreads), 0, s, a);
    if ((rc = hip_status(hipGetLastError(), "paged rotate launch")) != TC_OK) return rc;
  }
  return TC_OK;
}

}  // extern "C"
