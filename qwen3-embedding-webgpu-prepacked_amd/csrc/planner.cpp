// planner.cpp -- the attention operator's host planner (declared in planner.h): cost model,
// per-XCD slot assignment with split-K, and the launch arguments.
#include "planner.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <utility>
#include <vector>

namespace qattn {

int64_t pairs_of(int64_t L, const MaskSpec& m) {
  if (L <= 0) return 0;
  if (m.kind == 0) return L * (L + 1) / 2;
  int64_t total = 0;
  const int64_t ps = std::min<int64_t>(L, m.prefix), ws = std::min<int64_t>(L, m.window);
  for (int64_t q = 0; q < L; ++q) {
    // keys [0, min(q, ps-1)] U [max(0, q-ws+1), q]
    const int64_t a = std::min<int64_t>(q + 1, ps);    // prefix part
    const int64_t wlo = std::max<int64_t>(0, q - ws + 1);
    const int64_t b = q + 1 - std::max<int64_t>(wlo, a);  // window part not already counted
    total += a + std::max<int64_t>(0, b);
  }
  return total;
}

namespace {

// Cost model for load balancing, in quarter tiles (one 64-key tile of an entry = 4), fitted to
// the measured duration of every workgroup of the 16x500 and 1x5000 benchmark launches (start
// and end s_memtime of each workgroup of an instrumented build, 28 HBM-resident layers; least
// squares over 1024 workgroups, residual 2.6%):
//   duration = speed x (tiles + 3.3 entries + 4.6) tile times,
// speed 1 for the first workgroup of a CU and 1.3 for the second (the CUs issue from their
// oldest wavefronts first).  An entry's start and end (Q and first K tiles, last PV, O stores)
// cost about three tiles that the pipeline does not hide, a workgroup's start (all launch
// together, so their first loads queue at HBM) and end about four and a half, and a chunk of a
// split item no more than any other entry.  Refits on other plans gave 2.2-3.3 tiles per entry
// and 1.2-1.3 for the second workgroup (16x500: 37.5 us with the previous 0.75-tile entries and
// 1.2 factor, 35.6 us with 3.25-tile entries and 1.3).  Per-slot timelines of the current kernel
// put the second workgroup at 1.6x the first per tile and 1.26x per entry; among factors 1.3-1.6
// and entries of 2.75-3.75 tiles, 1.4 and 3.5 measured fastest (interleaved A/B: 16x500 -0.9%,
// 4x5000 -0.5%, the other launches within 0.3%).
constexpr int kEntryCost = 14;
int item_cost(int ntiles) { return 4 * ntiles + kEntryCost; }
constexpr int kSlotBase = 18;
constexpr int kChunkExtra = 0;
constexpr int kMinChunkTiles = 2;
// The merge kernel that follows a launch with split items (about 5 us, in cost units of a first
// slot): a split plan must beat the best unsplit plan by more than this.
constexpr int kMergeCost = 10;
// Slot speeds, in time per unit of cost (per mille): slots cu_count..2*cu_count-1 (an XCD's
// first 32 workgroups take one CU each) are the second workgroups.
constexpr int64_t kFirstSlotTime = 1000;
constexpr int64_t kSecondSlotTime = 1400;

}  // namespace

void plan_work(const qattn_run_desc* d, int max_slots, Plan* out, qattn_run_info* info_out,
               MaskSpec* mask_out) {
  if (max_slots < kXcds) max_slots = kXcds;
  const MaskSpec mask{d->mask, d->mask == QATTN_MASK_PREFIX_LOCAL ? d->prefix : 0,
                      d->mask == QATTN_MASK_PREFIX_LOCAL ? d->window : 0};
  struct Item {
    WorkItem w;
    int ntiles;
    int order;  // position in sequence-major order (sequence, then query block)
  };
  std::vector<Item> group_items[kXcds];
  qattn_run_info info{};
  info.block_queries = kBlockQ;
  for (int32_t s = 0; s < d->nseq; ++s) {
    const int start = d->cu_seqlens[s];
    const int L = d->cu_seqlens[s + 1] - start;
    info.tokens += L;
    info.pairs += pairs_of(L, mask);
    for (int qb = 0; qb * kBlockQ < L; ++qb) {
      const int q0 = qb * kBlockQ, q1 = std::min(L, q0 + kBlockQ) - 1;
      const TileRanges tr = key_tiles(q0, q1, L, mask);
      // MFMA tile work of one query head: the wavefronts holding rows [q0, q0+31] and
      // [q0+32, q0+63] each compute every tile of the work item.
      info.tile_pairs += (int64_t)tr.count() * (q0 + kWaveQ < L ? 2 : 1) * kWaveQ * kTileK;
      for (int g = 0; g < kKVHeads; ++g)
        group_items[g % kXcds].push_back({WorkItem{start, L, qb, (s << 4) | g, 0, tr.count(), -1, 0}, tr.count(),
                                          (int)group_items[g % kXcds].size()});
      ++info.work_items;
    }
  }
  info.work_items *= kKVHeads;
  // Per XCD group, longest processing time first with split-K: items in falling cost (stable,
  // so equal items keep sequence order) each go whole to the least loaded slot if that keeps it
  // within a target makespan T; otherwise the item is cut into chunks of key tiles that fill the
  // least loaded slots up to T (the chunks' partial softmax states are merged by a second
  // kernel).  T is scanned upward from the mean load; the plan with the smallest
  // makespan (then fewest chunks) wins.
  const int per_group = max_slots / kXcds;
  const bool may_split = !(d->flags & QATTN_FLAG_BATCH_INVARIANT);
  std::vector<std::vector<WorkItem>> lists[kXcds];
  int used = 0;
  for (int g = 0; g < kXcds; ++g) {
    auto& items = group_items[g];
    std::stable_sort(items.begin(), items.end(), [](const Item& a, const Item& b) { return a.ntiles > b.ntiles; });
    const int m = std::min<int>(per_group, (int)items.size());
    if (!m) continue;
    int64_t total = 0;  // the group's cost, workgroup bases included
    int max_tiles = 0;
    for (const Item& it : items) {
      total += item_cost(it.ntiles);
      max_tiles = std::max(max_tiles, it.ntiles);
    }
    total += (int64_t)m * kSlotBase;
    // Slot j of this group is global slot kXcds * j + g: the first half of the group's share
    // of the launch are first workgroups on their CUs.  Loads are in cost units; finish times
    // (load x time per unit) are what the plans balance.
    const int first_slots = std::max(1, per_group / kBlocksPerCU);
    std::vector<int64_t> slot_time(m);
    for (int j = 0; j < m; ++j) slot_time[j] = j < first_slots ? kFirstSlotTime : kSecondSlotTime;
    auto span_of = [&](const std::vector<int64_t>& load) {
      int64_t span = 0;
      for (int j = 0; j < m; ++j) span = std::max(span, load[j] * slot_time[j]);
      return span;
    };
    // One greedy pass for target finish time T: per item, (slot, tile range) pieces; returns the
    // makespan.
    struct Piece {
      int slot, item, a, b, cost;
    };
    auto greedy = [&](int64_t T, std::vector<Piece>* pieces, int* nchunks) {
      std::vector<int64_t> load(m, kSlotBase);
      // One min-heap of (load, slot) per speed class: within a class the least loaded slot
      // both finishes first and has the most room under T.
      typedef std::pair<int64_t, int> Entry;
      std::vector<Entry> heap[2];
      for (int j = 0; j < m; ++j) heap[j < first_slots ? 0 : 1].push_back({0, j});
      auto cmp = [](const Entry& x, const Entry& y) { return x > y; };
      for (auto& h : heap) std::make_heap(h.begin(), h.end(), cmp);
      auto top = [&](int c) { return heap[c].empty() ? -1 : heap[c].front().second; };
      auto take_out = [&](int j) {
        auto& h = heap[j < first_slots ? 0 : 1];
        std::pop_heap(h.begin(), h.end(), cmp);
        h.pop_back();
      };
      auto put_back = [&](int j) {
        auto& h = heap[j < first_slots ? 0 : 1];
        h.push_back({load[j], j});
        std::push_heap(h.begin(), h.end(), cmp);
      };
      // The class top that finishes first after adding cost c.
      auto earliest = [&](int64_t c) {
        const int a = top(0), b = top(1);
        if (a < 0) return b;
        if (b < 0) return a;
        return (load[a] + c) * slot_time[a] <= (load[b] + c) * slot_time[b] ? a : b;
      };
      // Room under T (cost units) of slot j.
      auto room = [&](int j) { return T / slot_time[j] - load[j]; };
      pieces->clear();
      *nchunks = 0;
      for (int i = 0; i < (int)items.size(); ++i) {
        const int n = items[i].ntiles;
        int j = earliest(item_cost(n));
        if ((load[j] + item_cost(n)) * slot_time[j] <= T || n < 2 * kMinChunkTiles || !may_split) {
          take_out(j);
          load[j] += item_cost(n);
          pieces->push_back({j, i, 0, n, item_cost(n)});
          put_back(j);
          continue;
        }
        std::vector<Piece> mine;
        int a = 0;
        while (a < n) {
          const int rest = n - a;
          // The class top with the most room under T takes a chunk that fills it; if no
          // slot has room for a chunk, the rest goes whole to the slot that finishes it first.
          const int x = top(0), y = top(1);
          j = x < 0 ? y : y < 0 ? x : (room(x) >= room(y) ? x : y);
          int take = (int)((room(j) - kEntryCost - kChunkExtra) / 4);
          if (take < kMinChunkTiles || (int)mine.size() == kMaxChunks - 1 || take >= rest ||
              rest - take < kMinChunkTiles) {
            take = rest;
            j = earliest(item_cost(rest) + kChunkExtra);
          }
          take_out(j);
          mine.push_back({j, i, a, a + take, item_cost(take) + kChunkExtra});
          load[j] += item_cost(take) + kChunkExtra;
          put_back(j);
          a += take;
        }
        if (mine.size() == 1) {  // not split after all
          load[mine[0].slot] -= kChunkExtra;
          mine[0].cost -= kChunkExtra;
        } else {
          *nchunks += (int)mine.size();
        }
        pieces->insert(pieces->end(), mine.begin(), mine.end());
      }
      return span_of(load);
    };
    // Rounds plan (whole items, for L2 locality): items in sequence-major order, m per round,
    // so the slots of an XCD work on the same few sequences at a time; within a round the
    // heaviest items go to the slots that would finish first.
    auto rounds = [&](std::vector<Piece>* pieces) {
      std::vector<int> seq_order(items.size());
      for (int i = 0; i < (int)items.size(); ++i) seq_order[items[i].order] = i;
      std::vector<int64_t> load(m, kSlotBase);
      std::vector<int> slot_ix(m);
      pieces->clear();
      for (size_t r0 = 0; r0 < seq_order.size(); r0 += m) {
        std::vector<int> its(seq_order.begin() + r0, seq_order.begin() + std::min(seq_order.size(), r0 + m));
        std::stable_sort(its.begin(), its.end(), [&](int a, int b) { return items[a].ntiles > items[b].ntiles; });
        for (int j = 0; j < m; ++j) slot_ix[j] = j;
        std::stable_sort(slot_ix.begin(), slot_ix.end(), [&](int a, int b) {
          return (load[a] + 1) * slot_time[a] < (load[b] + 1) * slot_time[b];
        });
        for (size_t k = 0; k < its.size(); ++k) {
          const int j = slot_ix[k];
          pieces->push_back({j, its[k], 0, items[its[k]].ntiles, item_cost(items[its[k]].ntiles)});
          load[j] += item_cost(items[its[k]].ntiles);
        }
      }
      return span_of(load);
    };
    // Local search on a plan.  Slots are visited from the one that finishes last; a slot hands
    // one of its pieces to a slot that finishes earlier, or trades it for a cheaper piece there,
    // when both then finish before it did.  Each move lowers the sorted vector of finish times
    // lexicographically, so the search ends; the first slots' moves lower the makespan, the
    // others make room for later ones.  Pieces only change slots: their order (each slot's
    // entry order and the chunk order of split items) stays.
    auto improve = [&](std::vector<Piece>* pieces) {
      std::vector<int64_t> load(m, kSlotBase);
      std::vector<std::vector<int>> held(m);
      for (int k = 0; k < (int)pieces->size(); ++k) {
        load[(*pieces)[k].slot] += (*pieces)[k].cost;
        held[(*pieces)[k].slot].push_back(k);
      }
      auto fin = [&](int j, int64_t l) { return l * slot_time[j]; };
      std::vector<int> order(m);
      for (int moves = 0; moves < 8 * (int)pieces->size(); ++moves) {
        for (int j = 0; j < m; ++j) order[j] = j;
        std::sort(order.begin(), order.end(), [&](int a, int b) { return fin(a, load[a]) > fin(b, load[b]); });
        bool moved = false;
        for (int oj = 0; oj < m && !moved; ++oj) {
          const int j = order[oj];
          const int64_t fj = fin(j, load[j]);
          for (int ok = m - 1; ok > oj && !moved; --ok) {
            const int k = order[ok];
            if (fin(k, load[k]) >= fj) break;
            for (int pi : held[j]) {
              const int cp = (*pieces)[pi].cost;
              int qsel = -1;
              bool ok_move = std::max(fin(j, load[j] - cp), fin(k, load[k] + cp)) < fj;
              if (!ok_move) {
                for (int qi : held[k]) {
                  const int cq = (*pieces)[qi].cost;
                  if (cq < cp && std::max(fin(j, load[j] - cp + cq), fin(k, load[k] - cq + cp)) < fj) {
                    qsel = qi;
                    break;
                  }
                }
                if (qsel < 0) continue;
              }
              auto relocate = [&](int idx, int from, int to) {
                held[from].erase(std::find(held[from].begin(), held[from].end(), idx));
                held[to].push_back(idx);
                (*pieces)[idx].slot = to;
                load[from] -= (*pieces)[idx].cost;
                load[to] += (*pieces)[idx].cost;
              };
              relocate(pi, j, k);
              if (qsel >= 0) relocate(qsel, k, j);
              moved = true;
              break;
            }
          }
        }
        if (!moved) break;
      }
      return span_of(load);
    };
    std::vector<Piece> best, trial;
    int64_t best_span = rounds(&best);
    best_span = improve(&best);
    int best_chunks = 0;
    int64_t best_eff = best_span;  // makespan plus the merge kernel when the plan splits
    // Lower bound of the makespan: the total cost spread over the slots in proportion to their
    // speeds.  Targets step by a quarter tile (one cost unit) on a first slot.
    double rate = 0.0;
    for (int j = 0; j < m; ++j) rate += 1.0 / (double)slot_time[j];
    const int64_t lo = (int64_t)std::ceil((double)total / rate);
    // LPT (whole items), then makespan-targeted split-K plans; a plan must be strictly better
    // than the rounds plan to replace it.
    for (int64_t T = lo; T <= lo + (4 * max_tiles + 8) * kFirstSlotTime && best_span > lo; T += kFirstSlotTime) {
      int nch = 0;
      const int64_t span = greedy(may_split ? T : INT64_MAX / 4, &trial, &nch);
      const int64_t eff = span + (nch ? (int64_t)kMergeCost * kFirstSlotTime : 0);
      if (eff < best_eff || (eff == best_eff && nch < best_chunks)) {
        best_span = span;
        best_eff = eff;
        best_chunks = nch;
        best.swap(trial);
      }
      if (!may_split) break;
    }
    best_span = improve(&best);
    // Emit: per slot in assignment order; chunks of one item share a split id and partials.
    lists[g].assign(m, {});
    for (size_t k = 0; k < best.size();) {
      size_t e = k + 1;
      while (e < best.size() && best[e].item == best[k].item) ++e;
      const WorkItem base = items[best[k].item].w;
      const int nch = (int)(e - k);
      const int split = nch > 1 ? out->splits++ : -1;
      const int first = nch > 1 ? out->partials : 0;
      if (nch > 1) out->partials += nch;
      for (size_t c = k; c < e; ++c) {
        WorkItem w = base;
        w.tile_begin = best[c].a;
        w.tile_end = best[c].b;
        w.split = split;
        w.part = nch > 1 ? (int)(c - k) | (nch << 4) | (first << 8) : 0;
        if (nch > 1 && c == k) out->split_heads.push_back(w);
        lists[g][best[c].slot].push_back(w);
      }
      k = e;
    }
    used = std::max(used, m);
  }
  out->items.clear();
  out->slot_begin.assign(1, 0);
  for (int j = 0; j < used; ++j)
    for (int g = 0; g < kXcds; ++g) {
      if (j < (int)lists[g].size())
        for (const WorkItem& w : lists[g][j]) out->items.push_back(w);
      out->slot_begin.push_back((int32_t)out->items.size());
    }
  info.slots = (int32_t)out->slot_begin.size() - 1;
  info.split_items = out->splits;
  info.flops = 4ll * kHeadDim * kQHeads * info.pairs;
  info.bytes = 12288ll * info.tokens + (d->o_last ? 4096ll * d->nseq : 0);
  if (info_out) *info_out = info;
  if (mask_out) *mask_out = mask;
}

void fill_params(AttnParams* p, const qattn_run_desc* d, const MaskSpec& mask, int32_t slots, const void* plan,
                 size_t items_bytes, size_t heads_bytes) {
  p->q = static_cast<const half_t*>(d->q);
  p->k = static_cast<const half_t*>(d->k);
  p->v = static_cast<const half_t*>(d->v) + d->v_offset;
  p->o = static_cast<half_t*>(d->o);
  p->o_last = static_cast<half_t*>(d->o_last);
  // Byte strides fit 32 bits: (L + 64) * stride * 2 < 2^31 is validated for every sequence.
  p->q_stride_b = (uint32_t)(d->q_row_stride * 2);
  p->k_stride_b = (uint32_t)(d->k_row_stride * 2);
  p->v_stride_b = (uint32_t)(d->v_row_stride * 2);
  p->o_stride_b = (uint32_t)(d->o_row_stride * 2);
  p->work = static_cast<const WorkItem*>(plan);
  p->splits = reinterpret_cast<const WorkItem*>(static_cast<const char*>(plan) + items_bytes);
  p->slot_begin = reinterpret_cast<const int32_t*>(static_cast<const char*>(plan) + items_bytes + heads_bytes);
  p->n_slots = slots;
  p->mask = mask;
  p->scale_log2 = (float)(1.4426950408889634 / std::sqrt(128.0));
}


}  // namespace qattn
