// Host planner of the prefix-tree decode (mentat_tree_decode and its counted
// variant): the segment, work-item and partial-slot plan of
// mentat_amd/tree_plan.py:build_plan, in native code so that a rollout's
// decode step can plan every step without holding up the GPU.
//
// Segments: lcp[i] = leading pages on which queries i - 1 and i hold the same
// block id with the same number of valid tokens (a shared partial page ends
// the run). A fork copies its parent's ids (core/paged_kv_cache.py:152-170),
// so in the depth-first leaf order (core/generator_utils.py:171-189) the
// queries holding a page are consecutive: page p of query i is shared by
// i .. j exactly when lcp[k] > p for i < k <= j. Each query's pages past
// lcp[i] are cut where that run of neighbours gets shorter.
//
// Items (int32 x 8, the kernel's layout): table row, first tile, tile count,
// valid tokens, kv head, member count, first slot, member offset. Shared tasks
// (segments of >= shared_min_groups groups of 16/G queries) come first, in
// chunks of shared_chunk_tiles tiles and member sets of 8 * 16/G, longest
// (most tiles) first and otherwise in the order below; then solo
// items in chunks of chunk_tiles tiles and sets of 16/G; both chunk-major,
// then kv head, then member set. Member j of an item writes slot first + j;
// q_slots lists each (query, head)'s slots in slot order.
#include <algorithm>
#include <cstdint>
#include <vector>

#include "mentat_capi.h"

namespace {

struct Seg {
  int owner, first_page, end_page, count;
};

constexpr int kFields = 8;
constexpr int kWavesPerTask = 8;  // member groups of one shared task
constexpr int kSharedMaxTiles = 32;

}  // namespace

extern "C" int mentat_tree_plan(const int32_t* tables, int64_t table_stride, const int32_t* qrows,
                                const int32_t* lens, int N, int block_size, int Hkv, int G, int chunk_tiles,
                                int shared_chunk_tiles, int shared_min_groups, int share, int32_t* counts,
                                int32_t* items, int max_shared, int max_solo, int32_t* members,
                                int32_t* q_slot_offsets, int32_t* q_slots, int max_slots) {
  if (N < 0 || !counts || !q_slot_offsets || Hkv <= 0 || G < 1 || 16 % G || block_size < 16 || block_size % 16 ||
      chunk_tiles < 1 || shared_chunk_tiles < 1 || shared_chunk_tiles > kSharedMaxTiles || table_stride <= 0 ||
      max_shared < 0 || max_solo < 0 || max_slots < 0)
    return MENTAT_EINVAL;
  if (N > 0 && (!tables || !qrows || !lens || (max_shared + max_solo > 0 && !items) || (max_slots > 0 &&
                                                                                     (!members || !q_slots))))
    return MENTAT_EINVAL;
  const int B = block_size, tpp = B / 16;
  std::vector<int> npg(N), lcp(N, 0);
  for (int i = 0; i < N; ++i) {
    const int n = std::max(lens[i], 0);
    npg[i] = (n + B - 1) / B;
    if (npg[i] > table_stride) return MENTAT_EINVAL;
  }
  if (share) {
    for (int i = 1; i < N; ++i) {
      const int32_t* ta = tables + (int64_t)qrows[i - 1] * table_stride;
      const int32_t* tb = tables + (int64_t)qrows[i] * table_stride;
      const int lim = std::min(npg[i - 1], npg[i]);
      int p = 0;
      while (p < lim) {
        const int va = std::min(B, lens[i - 1] - p * B), vb = std::min(B, lens[i] - p * B);
        if (ta[p] != tb[p] || va != vb) break;
        ++p;
        if (va < B) break;
      }
      lcp[i] = p;
    }
  }
  std::vector<Seg> segs;
  segs.reserve(2 * (size_t)N);
  for (int i = 0; i < N; ++i) {
    const int lo = lcp[i];
    int hi = npg[i];
    if (hi <= lo) continue;
    int j = i + 1;
    for (; j < N && lcp[j] > lo; ++j) {
      if (lcp[j] < hi) {
        segs.push_back({i, lcp[j], hi, j - i});  // pages [lcp[j], hi) of queries i .. j - 1
        hi = lcp[j];
      }
    }
    segs.push_back({i, lo, hi, j - i});
  }
  const int mg = 16 / G;
  int n_items[2] = {0, 0}, n_slots = 0;
  // pass 0: shared tasks (collected, then longest first: a stable sort by tile
  // count, so the kernel's queue starts the longest ones first), pass 1: solo items
  struct Rec {
    int row, c0, nt, end, h, mc, m0;
  };
  std::vector<Rec> recs;
  for (int pass = 0; pass < 2; ++pass) {
    const int chunk = pass == 0 ? shared_chunk_tiles : chunk_tiles;
    const int cap = pass == 0 ? kWavesPerTask * mg : mg;
    recs.clear();
    for (const Seg& s : segs) {
      const bool shared = (s.count + mg - 1) / mg >= shared_min_groups;
      if (shared != (pass == 0)) continue;
      const int end = std::min(s.end_page * B, std::max(lens[s.owner], 0));
      const int t0 = s.first_page * tpp, t1 = (end + 15) / 16;
      const int row = qrows[s.owner];
      for (int c0 = t0; c0 < t1; c0 += chunk) {
        const int nt = std::min(chunk, t1 - c0);
        for (int h = 0; h < Hkv; ++h)
          for (int k0 = 0; k0 < s.count; k0 += cap) recs.push_back({row, c0, nt, end, h, std::min(cap, s.count - k0),
                                                                   s.owner + k0});
      }
    }
    if (pass == 0)
      std::stable_sort(recs.begin(), recs.end(), [](const Rec& a, const Rec& b) { return a.nt > b.nt; });
    const int max_items = pass == 0 ? max_shared : max_solo;
    for (const Rec& r : recs) {
      if (n_items[pass] >= max_items || n_slots + r.mc > max_slots) return MENTAT_ESPACE;
      int32_t* it = items + (int64_t)(pass == 0 ? n_items[0] : max_shared + n_items[1]) * kFields;
      it[0] = r.row; it[1] = r.c0; it[2] = r.nt; it[3] = r.end; it[4] = r.h; it[5] = r.mc; it[6] = n_slots;
      it[7] = n_slots;
      for (int m = 0; m < r.mc; ++m) members[n_slots + m] = r.m0 + m;
      ++n_items[pass];
      n_slots += r.mc;
    }
  }
  // Solo items follow the shared tasks directly.
  if (n_items[0] < max_shared && n_items[1] > 0)
    std::copy(items + (int64_t)max_shared * kFields, items + (int64_t)(max_shared + n_items[1]) * kFields,
              items + (int64_t)n_items[0] * kFields);
  // q_slots: a stable counting sort of the slots by (query, head).
  const int nk = N * Hkv;
  std::fill(q_slot_offsets, q_slot_offsets + nk + 1, 0);
  std::vector<int> head_of(n_slots);
  for (int i = 0; i < n_items[0] + n_items[1]; ++i) {
    const int32_t* it = items + (int64_t)i * kFields;
    for (int m = 0; m < it[5]; ++m) head_of[it[6] + m] = it[4];
  }
  for (int sl = 0; sl < n_slots; ++sl) ++q_slot_offsets[members[sl] * Hkv + head_of[sl] + 1];
  for (int k = 0; k < nk; ++k) q_slot_offsets[k + 1] += q_slot_offsets[k];
  std::vector<int> fill(q_slot_offsets, q_slot_offsets + nk);
  for (int sl = 0; sl < n_slots; ++sl) q_slots[fill[members[sl] * Hkv + head_of[sl]]++] = sl;
  counts[0] = n_items[0];
  counts[1] = n_items[1];
  counts[2] = n_slots;
  return MENTAT_OK;
}
