// Byte-level BPE tokenizer (host code): training and encoding.
//
// Reference behaviour: simple-llm/src/common/bpe_tokenizer.c (a standalone C
// program the reference's Python wrapper, common/bpe_tokenizer.py, runs as a
// subprocess):
//  * train (bpe_tokenizer.c:155-243): ids = the corpus bytes; each round
//    counts every adjacent pair (overlapping occurrences included), takes the
//    pair with the largest count, appends merge (p1, p2) -> 256 + round, and
//    replaces its occurrences left to right without overlap (:110-128). Ties
//    go to the first pair of the reference's hash-table traversal
//    (get_stats_fast, :30-84): buckets (p1 * 2654435761 + p2) mod 10007 in
//    ascending order, and inside a bucket the most recently inserted pair
//    first -- the one whose first occurrence in this round's sequence is
//    latest. At most vocab_size - 256 (<= 49744) rounds; training stops early
//    when no pair is left.
//  * encode (:246-355): one pass; at each position, if the two raw bytes
//    form a merge, the first such merge in file order replaces them,
//    otherwise the byte is emitted. Merges involving merged ids never apply
//    here, as in the reference.
//
// Design: the pair counts of a round go into a flat open-addressing table
// sized to the distinct pairs (no per-entry allocation), recording each pair's
// count and first position as it is met, so the winner and its tie-break
// come from one scan of the table. Encoding uses a 256 x 256 table of the
// first merge of each byte pair.
#include <algorithm>
#include <cstdint>
#include <vector>

#include "skv.h"

namespace skv {
int set_error(int code, const char* fmt, ...);  // skv_api.hip: skv_last_error's text
}

namespace {

constexpr int kRefMaxVocab = 50000;  // MAX_VOCAB_SIZE of the reference
constexpr uint32_t kRefBuckets = 10007;

int fail(int code, const char* msg) { return skv::set_error(code, "%s", msg); }

inline uint32_t ref_bucket(int p1, int p2) {
  return ((uint32_t)p1 * 2654435761u + (uint32_t)p2) % kRefBuckets;
}

// Pair counts of one round: open addressing, grown by doubling at half load,
// so its size follows the distinct pairs (thousands for text) rather than
// the sequence length, and clearing it each round is cheap.
struct PairTable {
  std::vector<uint64_t> key;  // (p1 << 32 | p2) + 1; 0 = empty
  std::vector<int32_t> count;
  std::vector<int64_t> first;
  uint64_t mask = 0;
  size_t used = 0;

  void reset() {
    if (key.empty()) alloc(1 << 14);
    std::fill(key.begin(), key.end(), 0);
    used = 0;
  }
  void alloc(size_t cap) {
    key.assign(cap, 0);
    count.assign(cap, 0);
    first.assign(cap, 0);
    mask = cap - 1;
  }
  static uint64_t mix(uint64_t k) {
    k ^= k >> 33;
    k *= 0xff51afd7ed558ccdull;
    k ^= k >> 33;
    return k;
  }
  void insert(uint64_t k, int32_t c, int64_t f) {
    uint64_t h = mix(k) & mask;
    while (key[h] != 0) h = (h + 1) & mask;
    key[h] = k;
    count[h] = c;
    first[h] = f;
  }
  void grow() {
    std::vector<uint64_t> k0;
    std::vector<int32_t> c0;
    std::vector<int64_t> f0;
    k0.swap(key);
    c0.swap(count);
    f0.swap(first);
    alloc(k0.size() * 2);
    for (size_t h = 0; h < k0.size(); ++h)
      if (k0[h] != 0) insert(k0[h], c0[h], f0[h]);
  }
  void add(int p1, int p2, int64_t pos) {
    const uint64_t k = (((uint64_t)(uint32_t)p1 << 32) | (uint32_t)p2) + 1;
    uint64_t h = mix(k) & mask;
    while (key[h] != 0 && key[h] != k) h = (h + 1) & mask;
    if (key[h] == k) {
      ++count[h];
      return;
    }
    key[h] = k;
    count[h] = 1;
    first[h] = pos;
    if (++used * 2 > key.size()) grow();
  }
};

}  // namespace

extern "C" int skv_bpe_train(const uint8_t* corpus, size_t n, int vocab_size, int32_t* merges,
                             int max_merges, int* n_merges) {
  if (!n_merges || (n > 0 && !corpus)) return fail(SKV_E_INVALID, "skv_bpe_train: null pointer");
  *n_merges = 0;
  int rounds = vocab_size - 256;
  if (rounds > kRefMaxVocab - 256) rounds = kRefMaxVocab - 256;
  if (rounds <= 0) return SKV_OK;
  if (!merges || max_merges < rounds)
    return fail(SKV_E_INVALID, "skv_bpe_train: merges buffer smaller than vocab_size - 256");
  std::vector<int32_t> ids(corpus, corpus + n);
  PairTable tab;
  for (int r = 0; r < rounds; ++r) {
    const int64_t len = (int64_t)ids.size();
    if (len < 2) break;
    tab.reset();
    for (int64_t i = 0; i + 1 < len; ++i) tab.add(ids[i], ids[i + 1], i);
    // winner: largest count; then lowest reference bucket; then latest first
    // occurrence (the reference's chain holds the latest insertion first)
    int best_c = -1, bp1 = 0, bp2 = 0;
    uint32_t best_b = 0;
    int64_t best_first = -1;
    for (size_t h = 0; h < tab.key.size(); ++h) {
      if (tab.key[h] == 0) continue;
      const uint64_t k = tab.key[h] - 1;
      const int p1 = (int)(k >> 32), p2 = (int)(uint32_t)k;
      const int c = tab.count[h];
      const uint32_t b = ref_bucket(p1, p2);
      const bool better = c > best_c || (c == best_c && (b < best_b ||
                                                        (b == best_b && tab.first[h] > best_first)));
      if (better) {
        best_c = c;
        best_b = b;
        best_first = tab.first[h];
        bp1 = p1;
        bp2 = p2;
      }
    }
    const int new_id = 256 + r;
    merges[3 * r + 0] = bp1;
    merges[3 * r + 1] = bp2;
    merges[3 * r + 2] = new_id;
    *n_merges = r + 1;
    // left to right, non-overlapping replacement, in place
    int64_t o = 0;
    for (int64_t i = 0; i < len;) {
      if (i + 1 < len && ids[i] == bp1 && ids[i + 1] == bp2) {
        ids[o++] = new_id;
        i += 2;
      } else {
        ids[o++] = ids[i++];
      }
    }
    ids.resize(o);
  }
  return SKV_OK;
}

extern "C" int skv_bpe_encode(const uint8_t* text, size_t n, const int32_t* merges, int n_merges,
                              int32_t* ids, size_t* n_ids) {
  if (!n_ids || (n > 0 && (!text || !ids)) || (n_merges > 0 && !merges))
    return fail(SKV_E_INVALID, "skv_bpe_encode: null pointer");
  if (n_merges < 0) return fail(SKV_E_INVALID, "skv_bpe_encode: n_merges < 0");
  // first merge (in order) of each pair of raw bytes
  std::vector<int32_t> first(256 * 256, -1);
  const int m = n_merges < kRefMaxVocab ? n_merges : kRefMaxVocab;  // the reference reads <= 50000
  for (int j = 0; j < m; ++j) {
    const int p1 = merges[3 * j], p2 = merges[3 * j + 1];
    if (p1 >= 0 && p1 < 256 && p2 >= 0 && p2 < 256 && first[p1 * 256 + p2] < 0)
      first[p1 * 256 + p2] = merges[3 * j + 2];
  }
  size_t o = 0;
  for (size_t i = 0; i < n;) {
    if (i + 1 < n) {
      const int id = first[text[i] * 256 + text[i + 1]];
      if (id >= 0) {
        ids[o++] = id;
        i += 2;
        continue;
      }
    }
    ids[o++] = text[i++];
  }
  *n_ids = o;
  return SKV_OK;
}
