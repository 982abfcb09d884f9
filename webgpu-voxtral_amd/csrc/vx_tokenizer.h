// vx_tokenizer.h -- byte-level BPE of the Tekken tokenizer (encoding only):
// TekkenTokenizer.bpeEncode, src/tokenizer.ts:196-249.  Host code.
//
// The reference merges one pair per pass: it scans all adjacent parts for
// the pair whose concatenation has the lowest vocabulary rank (the leftmost
// on equal ranks), merges it, and rescans -- O(n^2) per piece.  Here the
// parts form a linked list and the candidate pairs a min-heap keyed by
// (rank, position of the left part); entries made stale by a merge are
// skipped when popped.  The heap always yields the lowest-rank, leftmost
// pair among the current adjacent pairs, so the merge sequence, and the
// result, are the reference's.
#pragma once
#include <cstdint>
#include <queue>
#include <string>
#include <unordered_map>
#include <vector>

namespace vx {

class BpeVocab {
 public:
  BpeVocab(int32_t num_special) : num_special_(num_special) {}

  void add(const uint8_t *bytes, size_t len, int32_t rank) {
    rank_[std::string((const char *)bytes, len)] = rank;
  }
  size_t size() const { return rank_.size(); }

  // token ids of one pre-tokenized piece appended to out: rank + the number
  // of special tokens, or 0 (UNK) for a part the vocabulary lacks
  void encode(const uint8_t *p, size_t n, std::vector<int32_t> &out) const {
    if (n <= 1) {  // a single byte, or an empty piece (no part: UNK)
      out.push_back(n == 1 ? id_of(p, 1) : 0);
      return;
    }
    // part i covers bytes [start[i], start[next[i]]); prev/next link parts
    std::vector<int32_t> next(n), prev(n), len(n, 1), ver(n, 0);
    for (size_t i = 0; i < n; i++) {
      next[i] = (int32_t)i + 1;
      prev[i] = (int32_t)i - 1;
    }
    struct Cand {
      int32_t rank, left, ver_l, ver_r;
      bool operator>(const Cand &o) const {
        return rank != o.rank ? rank > o.rank : left > o.left;
      }
    };
    std::priority_queue<Cand, std::vector<Cand>, std::greater<Cand>> heap;
    auto push = [&](int32_t l) {
      const int32_t r = next[l];
      if (r >= (int32_t)n) return;
      const int32_t rk = rank_of(p + l, (size_t)(len[l] + len[r]));
      if (rk >= 0) heap.push({rk, l, ver[l], ver[r]});
    };
    for (int32_t i = 0; i + 1 < (int32_t)n; i++) push(i);
    while (!heap.empty()) {
      const Cand c = heap.top();
      heap.pop();
      const int32_t l = c.left, r = next[l];
      if (len[l] == 0 || r >= (int32_t)n || ver[l] != c.ver_l || ver[r] != c.ver_r) continue;
      // merge r into l
      len[l] += len[r];
      len[r] = 0;
      next[l] = next[r];
      if (next[r] < (int32_t)n) prev[next[r]] = l;
      ver[l]++;
      if (prev[l] >= 0) push(prev[l]);
      push(l);
    }
    for (int32_t i = 0; i < (int32_t)n; i = next[i]) out.push_back(id_of(p + i, (size_t)len[i]));
  }

 private:
  int32_t num_special_;
  std::unordered_map<std::string, int32_t> rank_;

  int32_t rank_of(const uint8_t *p, size_t n) const {
    auto it = rank_.find(std::string((const char *)p, n));
    return it == rank_.end() ? -1 : it->second;
  }
  int32_t id_of(const uint8_t *p, size_t n) const {
    const int32_t r = rank_of(p, n);
    return r < 0 ? 0 : r + num_special_;
  }
};

}  // namespace vx
