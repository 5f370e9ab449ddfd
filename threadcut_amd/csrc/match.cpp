// Split of a new request against the cached token sequence (host code).
//
// Same rule as threadcut/match.py:25-48: A = the longest common prefix capped
// at len(new) - 1; C = the longest run of the tokens after A that also starts
// somewhere in the cache after position a, found from a min_suffix-token
// anchor, first longest wins; D = the rest. The anchor search here is a
// Rabin-Karp rolling hash over the cache (one pass, each hash hit verified),
// instead of comparing every window, so it stays linear in the cache length.
#include <stdint.h>
#include <string.h>

#include <algorithm>

#include "../../include/threadcut_hip.h"

namespace {

int64_t common_prefix(const int64_t* x, int64_t nx, const int64_t* y, int64_t ny) {
  const int64_t n = std::min(nx, ny);
  int64_t i = 0;
  while (i < n && x[i] == y[i]) ++i;
  return i;
}

}  // namespace

extern "C" int tc_match_split(const int64_t* cached, int64_t n_cached, const int64_t* fresh, int64_t n_fresh,
                              int64_t min_suffix, int suffix, int64_t out[3]) {
  if (!out || n_cached < 0 || n_fresh < 0 || min_suffix < 0 || (n_cached > 0 && !cached) ||
      (n_fresh > 0 && !fresh))
    return TC_ERR_INVALID_ARGUMENT;
  const int64_t a = std::min(common_prefix(cached, n_cached, fresh, n_fresh), n_fresh - 1);
  out[0] = a;
  out[1] = a;
  out[2] = 0;
  // rest = fresh[a:]; a == -1 only for an empty request, whose rest is empty too.
  const int64_t* rest = fresh + std::max<int64_t>(a, 0);
  const int64_t n_rest = a < 0 ? 0 : n_fresh - a;
  if (!suffix || n_rest <= min_suffix || n_cached - (a + 1) < min_suffix) return TC_OK;

  const int64_t m = min_suffix;
  const int64_t lo = a + 1;                  // first candidate start
  const int64_t last = n_cached - m;         // last candidate start
  if (m == 0) {
    // Every start matches an empty anchor.
    for (int64_t j = lo; j <= last; ++j) {
      const int64_t c = std::min(common_prefix(cached + j, n_cached - j, rest, n_rest), n_rest - 1);
      if (c > out[2]) { out[1] = j; out[2] = c; }
    }
    return TC_OK;
  }
  // Polynomial hash mod 2^64 of a window; tokens are offset by one so 0 is not absorbing.
  const uint64_t base = 1000003ull;
  uint64_t top = 1;  // base^(m-1)
  for (int64_t i = 1; i < m; ++i) top *= base;
  uint64_t target = 0, h = 0;
  for (int64_t i = 0; i < m; ++i) {
    target = target * base + static_cast<uint64_t>(rest[i]) + 1u;
    h = h * base + static_cast<uint64_t>(cached[lo + i]) + 1u;
  }
  for (int64_t j = lo;; ++j) {
    if (h == target && memcmp(cached + j, rest, static_cast<size_t>(m) * sizeof(int64_t)) == 0) {
      const int64_t c = std::min(common_prefix(cached + j, n_cached - j, rest, n_rest), n_rest - 1);
      if (c > out[2]) { out[1] = j; out[2] = c; }
    }
    if (j == last) break;
    h = (h - (static_cast<uint64_t>(cached[j]) + 1u) * top) * base + static_cast<uint64_t>(cached[j + m]) + 1u;
  }
  return TC_OK;
}
