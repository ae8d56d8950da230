// attn_plan.cpp — how launch_attention splits the work of the partitioned
// (long-sequence and batch) attention kernels, and the scratch that split
// needs: host arithmetic only, shared by the launcher, the model's workspace
// sizing and the argument checks.
#include "internal.hpp"

namespace glypr {

// Queries per block: 16 AQS.  HD 512 runs one row of 16 queries (its two
// 32 KB tile slots and 192 accumulator registers per lane leave no room for
// more waves).  HD 256 takes 64-query blocks for long sequences and for many
// rows (a batch of sequences): from 4096 rows the 64-query blocks' four-fold
// K/V reuse beats the 16-query blocks' extra workgroups (32 x 512 rows:
// 64 against 116 us per layer; 16 x 512: 44 against 62 us), below it the
// 16-query blocks are as fast or faster (4 x 512: 24 against 30 us).
int attn_qs(int64_t T, int64_t rows, int64_t hd) {
  if (hd == 512) return 1;
  return T > ATTN_SMALL_T || rows >= ATTN_QS4_ROWS ? 4 : 1;
}

// Tseg: the longest sequence (its key range sets the tile count); rows: the
// padded rows of all sequences (they set the query blocks).
int attn_kb_per_part(int64_t Tseg, int64_t rows, int64_t hd, int64_t nq, int64_t nkv,
                     int64_t window, int* kparts) {
  const int64_t aqb = 16 * attn_qs(Tseg, rows, hd);
  const int64_t nqb = rows / aqb;
  int64_t nkb = (Tseg + ATTN_AK - 1) / ATTN_AK;
  if (window > 0 && Tseg > window) {
    int64_t band = (2 * window + aqb + ATTN_AK - 1) / ATTN_AK + 1;
    if (band < nkb) nkb = band;
  }
  int64_t want = (ATTN_BLOCKS + nqb * nkv - 1) / (nqb * nkv);
  if (want > (nkb + 1) / 2) want = (nkb + 1) / 2;
  if (want < (nkb + 63) / 64) want = (nkb + 63) / 64;
  if (want < 1) want = 1;
  const int64_t per = (nkb + want - 1) / want;
  *kparts = (int)((nkb + per - 1) / per);
  return (int)per;
}

bool attention_rows_ok(int64_t rows, int64_t hd) {
  return 2 * hd * attn_padded_len(rows) < (int64_t(1) << 31);
}

bool attention_supported(int64_t T, int64_t nq, int64_t nkv, int64_t hd, int64_t window) {
  if ((hd != 256 && hd != 512) || nq <= 0 || nkv <= 0 || nq % nkv != 0 || nq / nkv > 4)
    return false;
  if (T <= 0) return true;
  if (!attention_rows_ok(T, hd)) return false;
  int kparts;
  attn_kb_per_part(T, attn_padded_len(T), hd, nq, nkv, window, &kparts);
  return kparts <= 64;   // the combine holds one partition per lane
}

size_t attention_scratch_floats(int64_t T, int64_t nq, int64_t nkv, int64_t hd, int64_t window,
                                int64_t rows) {
  const int64_t tp = rows > 0 ? rows : attn_padded_len(T);
  int kp;
  attn_kb_per_part(T, tp, hd, nq, nkv, window, &kp);
  return (size_t)(kp * tp * nq * (hd + 2));
}

size_t attention_scratch_bound(int64_t max_t, int64_t cap_rows, int64_t nq, int64_t nkv,
                               int64_t hd, int64_t window) {
  // For one tk, kparts depends on rows only through the query blocks:
  // their count (want) and their size (16 or 64 queries, switching at
  // ATTN_QS4_ROWS).  Every row count is visited until neither can change
  // kparts any more: the blocks are 64 queries and they fill a round by
  // themselves (nqb nkv >= ATTN_BLOCKS, so want = 1 and kparts = the clamp
  // of the key tiles alone).  From there kparts is constant and the
  // product kparts * rows peaks at the capacity.
  size_t best = 0;
  for (int64_t tk = 32;; tk += 32) {
    if (tk > max_t) tk = max_t;
    for (int64_t rows = attn_padded_len(tk); rows <= cap_rows; rows += 64) {
      size_t sc = attention_scratch_floats(tk, nq, nkv, hd, window, rows);
      best = sc > best ? sc : best;
      const int64_t aqb = 16 * attn_qs(tk, rows, hd);
      if (rows >= ATTN_QS4_ROWS && (rows / aqb) * nkv >= ATTN_BLOCKS && rows < cap_rows) {
        sc = attention_scratch_floats(tk, nq, nkv, hd, window, cap_rows);
        best = sc > best ? sc : best;
        break;
      }
    }
    if (tk == max_t) break;
  }
  return best;
}

}  // namespace glypr
