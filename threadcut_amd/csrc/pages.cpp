// Page-table arithmetic of the paged KV cache (host code).
//
// A sequence's cache is a list of fragments, rows (page, first slot, count)
// of int64: count consecutive slots of one page holding consecutive logical
// tokens, the fragments in logical order. The kernels read a sequence as
// tiles of at most 16 rows of one page (the decode's tile table, the prune's
// rotation list) or through the byte offset of every token's row (the paged
// prefill); a prune keeps two logical ranges and frees the pages nothing
// kept uses. These loops replace per-call numpy work that cost tens of
// microseconds per prune in small-array overhead.
#include <stdint.h>

#include <algorithm>
#include <vector>

#include "../../include/threadcut_hip.h"

namespace {

constexpr int64_t kTile = 16;  // rows per tile (the decode kernel's wave tile)

// A fragment list is well formed when every fragment names a page id that
// fits 32 bits and count >= 1 slots that stay inside one page of page_tokens.
bool malformed(const int64_t* frags, int64_t num_frags, int64_t page_tokens) {
  if (num_frags < 0 || (num_frags > 0 && !frags) || page_tokens < 1 || page_tokens > INT32_MAX) return true;
  for (int64_t i = 0; i < num_frags; ++i) {
    const int64_t* f = frags + 3 * i;
    if (f[0] < 0 || f[0] > INT32_MAX || f[1] < 0 || f[2] < 1 || f[1] > page_tokens - f[2]) return true;
  }
  return false;
}

// Fragments covering logical tokens [lo, hi), appended to out.
void cut(const int64_t* frags, int64_t num_frags, int64_t lo, int64_t hi, std::vector<int64_t>& out) {
  int64_t begin = 0;
  for (int64_t i = 0; i < num_frags && begin < hi; ++i) {
    const int64_t* f = frags + 3 * i;
    const int64_t end = begin + f[2];
    const int64_t l = std::max(lo, begin), h = std::min(hi, end);
    if (l < h) {
      out.push_back(f[0]);
      out.push_back(f[1] + (l - begin));
      out.push_back(h - l);
    }
    begin = end;
  }
}

std::vector<int64_t> pages_of(const int64_t* frags, int64_t num_frags) {
  std::vector<int64_t> p(static_cast<size_t>(num_frags));
  for (int64_t i = 0; i < num_frags; ++i) p[i] = frags[3 * i];
  std::sort(p.begin(), p.end());
  p.erase(std::unique(p.begin(), p.end()), p.end());
  return p;
}

}  // namespace

extern "C" {

int64_t tc_page_tiles(const int64_t* frags, int64_t num_frags, int64_t page_tokens, int64_t first_pos, int32_t* tiles,
                      int64_t max_tiles) {
  if (malformed(frags, num_frags, page_tokens) || first_pos < 0 || max_tiles < 0) return -TC_ERR_INVALID_ARGUMENT;
  int64_t n = 0;
  for (int64_t i = 0; i < num_frags; ++i) {
    const int64_t s = frags[3 * i + 1], e = s + frags[3 * i + 2];
    n += (e - 1) / kTile + 1 - s / kTile;
  }
  if (!tiles || max_tiles < n) return n;
  int64_t pos = first_pos, k = 0;
  for (int64_t i = 0; i < num_frags; ++i) {
    const int64_t page = frags[3 * i], s = frags[3 * i + 1], e = s + frags[3 * i + 2];
    for (int64_t t = s / kTile; t * kTile < e; ++t) {
      const int64_t lo = std::max(s, t * kTile), hi = std::min(e, (t + 1) * kTile);
      if (pos > INT32_MAX) return -TC_ERR_INVALID_ARGUMENT;
      int32_t* o = tiles + 4 * k++;
      o[0] = static_cast<int32_t>(page);
      o[1] = static_cast<int32_t>(lo);
      o[2] = static_cast<int32_t>(hi - lo);
      o[3] = static_cast<int32_t>(pos);
      pos += hi - lo;
    }
  }
  return n;
}

int tc_page_prune(const int64_t* frags, int64_t num_frags, int64_t page_tokens, int64_t a, int64_t c0, int64_t c,
                  int64_t* kept, int64_t* suffix, int64_t* freed, int64_t counts[3]) {
  if (malformed(frags, num_frags, page_tokens) || !kept || !suffix || !freed || !counts) return TC_ERR_INVALID_ARGUMENT;
  int64_t n = 0;
  for (int64_t i = 0; i < num_frags; ++i) n += frags[3 * i + 2];
  if (a < 0 || c < 0 || c0 < a || c0 + c > n) return TC_ERR_INVALID_ARGUMENT;
  std::vector<int64_t> head, suf;
  cut(frags, num_frags, 0, a, head);
  cut(frags, num_frags, c0, c0 + c, suf);
  std::vector<int64_t> out(head);
  size_t from = 0;
  if (!head.empty() && !suf.empty()) {
    int64_t* last = out.data() + out.size() - 3;
    if (last[0] == suf[0] && last[1] + last[2] == suf[1]) {  // adjacent slots of one page merge back
      last[2] += suf[2];
      from = 3;
    }
  }
  out.insert(out.end(), suf.begin() + from, suf.end());
  const int64_t nk = static_cast<int64_t>(out.size() / 3), ns = static_cast<int64_t>(suf.size() / 3);
  std::copy(out.begin(), out.end(), kept);
  std::copy(suf.begin(), suf.end(), suffix);
  const std::vector<int64_t> before = pages_of(frags, num_frags), after = pages_of(out.data(), nk);
  const int64_t nf = std::set_difference(before.begin(), before.end(), after.begin(), after.end(), freed) - freed;
  counts[0] = nk;
  counts[1] = ns;
  counts[2] = nf;
  return TC_OK;
}

int64_t tc_page_token_offsets(const int64_t* frags, int64_t num_frags, int64_t page_tokens, int64_t page_bytes,
                              int64_t slot_bytes, int32_t* out, int64_t pitch) {
  if (malformed(frags, num_frags, page_tokens) || page_bytes < 0 || slot_bytes < 0 || pitch < 0 ||
      (pitch > 0 && !out))
    return -TC_ERR_INVALID_ARGUMENT;
  int64_t t = 0;
  for (int64_t i = 0; i < num_frags; ++i) {
    const int64_t page = frags[3 * i], s = frags[3 * i + 1], cnt = frags[3 * i + 2];
    if (t + cnt > pitch) return -TC_ERR_INVALID_ARGUMENT;
    const int64_t base = page * page_bytes;
    if (base + (s + cnt - 1) * slot_bytes > INT32_MAX) return -TC_ERR_INVALID_ARGUMENT;
    for (int64_t j = 0; j < cnt; ++j) out[t++] = static_cast<int32_t>(base + (s + j) * slot_bytes);
  }
  for (int64_t j = t; j < pitch; ++j) out[j] = INT32_MIN;
  return t;
}

}  // extern "C"
