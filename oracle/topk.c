/* Exact top-k selection of the DSA indexer, restated in plain C (test oracle only).
 *
 * Follows the reference's exact top-k (sgl_amd_mono/glm53/gfx950/kernel.py:3002-3636,
 * unpaged :2543-2682; order key :2698-2699; V4 ties deepseek_v4/gfx950/kernels/stages/
 * indexer.py:693-700): scores are ranked by the radix order key of their f32 bits
 * (bits >= 0 ? bits ^ 0x80000000 : ~bits, larger first); the selected set is every key
 * above the k-th largest key plus the lowest positions among the keys equal to it; the
 * output lists the selected positions in ascending position order.
 *
 * The threshold is found by a byte-wise radix select (four histogram passes), an
 * algorithm independent of the sort the tests compare it with. */
#include <stdint.h>
#include <string.h>

static inline uint32_t radix_key(float f) {
  uint32_t b;
  memcpy(&b, &f, 4);
  return (b & 0x80000000u) ? ~b : (b ^ 0x80000000u);
}

/* The k-th largest key of s[0..n) (1 <= k <= n). */
static uint32_t kth_key(const float* s, int n, int k) {
  uint32_t prefix = 0, mask = 0;
  int want = k; /* rank still to find inside the current prefix class */
  for (int shift = 24; shift >= 0; shift -= 8) {
    int hist[256] = {0};
    for (int i = 0; i < n; ++i) {
      uint32_t key = radix_key(s[i]);
      if ((key & mask) == prefix) hist[(key >> shift) & 255]++;
    }
    int d = 255;
    for (; d > 0; --d) {
      if (hist[d] >= want) break;
      want -= hist[d];
    }
    prefix |= (uint32_t)d << shift;
    mask |= 255u << shift;
  }
  return prefix;
}

/* Select min(n, k) positions of s[0..n); write them ascending to out; return the count. */
int oracle_topk(const float* s, int n, int k, int32_t* out) {
  if (n <= 0 || k <= 0) return 0;
  if (k >= n) {
    for (int i = 0; i < n; ++i) out[i] = i;
    return n;
  }
  const uint32_t thr = kth_key(s, n, k);
  int above = 0;
  for (int i = 0; i < n; ++i) above += radix_key(s[i]) > thr;
  int ties = k - above, m = 0;
  for (int i = 0; i < n; ++i) {
    uint32_t key = radix_key(s[i]);
    if (key > thr || (key == thr && ties-- > 0)) out[m++] = i;
  }
  return m;
}

/* Rows of a [rows, stride] score matrix, each over its first lens[r] entries; out is
 * [rows, k], entries past a row's count set to -1. */
void oracle_topk_rows(const float* s, int rows, int stride, const int32_t* lens, int k,
                      int32_t* out) {
  for (int r = 0; r < rows; ++r) {
    int32_t* o = out + (int64_t)r * k;
    int m = oracle_topk(s + (int64_t)r * stride, lens[r], k, o);
    for (int i = m; i < k; ++i) o[i] = -1;
  }
}
