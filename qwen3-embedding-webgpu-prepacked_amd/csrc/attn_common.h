// attn_common.h -- geometry, mask predicate, key-tile iterator and per-tile mask cases shared by
// the attention kernel, the debug-mask kernel and the host planner.  The kernel selects its
// element compares with tile_mask_case(); kept_keys_row() walks the same iteration with the same
// case rules, and the kernel's MASKBITS variant reports what its executed compares kept.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qattn {

constexpr int kHeadDim = 128;  // model.ts:18-23 (Q_WIDTH 2048 / 16 heads)
constexpr int kQHeads = 16;
constexpr int kKVHeads = 8;
constexpr int kGroup = kQHeads / kKVHeads;  // ops.ts:196 kv_head = q_head / 2

constexpr int kBlockQ = 64;   // query positions per work item (x 2 heads of one KV group)
constexpr int kTileK = 64;    // keys per LDS tile
constexpr int kWaveQ = 32;    // query positions per wavefront (one 32-row MFMA tile, one head)
constexpr int kWaves = kGroup * kBlockQ / kWaveQ;  // 4: 2 heads x 2 groups of 32 positions
constexpr int kThreads = kWaves * 64;

struct MaskSpec {
  int kind;    // 0 causal, 1 prefix + local window
  int prefix;  // reference 176
  int window;  // reference 432
};

// Reference predicate ops.ts:205-206,220, clamps included:
//   q < S && k <= q && k < S && (k < min(S,prefix) || k + min(S,window) > q)
// (the causal kind drops the last conjunct).
__host__ __device__ inline bool retained(int q, int k, int S, const MaskSpec& m) {
  if (!(q < S && k <= q && k < S)) return false;
  if (m.kind == 0) return true;
  const int ps = S < m.prefix ? S : m.prefix;
  const int ws = S < m.window ? S : m.window;
  return k < ps || k + ws > q;
}

// Key tiles that query rows [qa, qb] (0 <= qa <= qb < S) of one sequence must visit: at most two
// half-open ranges of tile indices.  Causal: keys <= qb.  Prefix/local: keys < min(S,prefix)
// plus keys >= qa - min(S,window) + 1; every key outside both is masked for every row in
// [qa, qb] (k + ws > q with q >= qa needs k >= qa - ws + 1), so skipping it is exact.
struct TileRanges {
  int b0, e0, b1, e1;
  __host__ __device__ int count() const { return (e0 - b0) + (e1 - b1); }
  __host__ __device__ int at(int i) const { return i < e0 - b0 ? b0 + i : b1 + (i - (e0 - b0)); }
};

__host__ __device__ inline TileRanges key_tiles(int qa, int qb, int S, const MaskSpec& m) {
  TileRanges r;
  const int last = qb / kTileK;
  r.b0 = 0;
  r.e0 = last + 1;
  r.b1 = 0;
  r.e1 = 0;
  if (m.kind == 0) return r;
  const int ps = S < m.prefix ? S : m.prefix;
  const int ws = S < m.window ? S : m.window;
  int pe = (ps + kTileK - 1) / kTileK;
  if (pe > last + 1) pe = last + 1;
  int wstart = qa - ws + 1;
  if (wstart < 0) wstart = 0;
  const int wb = wstart / kTileK;
  if (wb > pe) {
    r.e0 = pe;
    r.b1 = wb;
    r.e1 = last + 1;
  }
  return r;
}

// Is every key of the tile retained for every row in [qa, qb]?  Then no element mask is needed.
__host__ __device__ inline bool tile_full(int kb, int qa, int qb, int S, const MaskSpec& m) {
  const int ke = kb + kTileK - 1;
  if (ke > qa) return false;  // causal for the first row (ke <= qa < S also keeps keys in range)
  if (m.kind == 0) return true;
  const int ps = S < m.prefix ? S : m.prefix;
  const int ws = S < m.window ? S : m.window;
  return ke < ps || qb - kb < ws;
}

// Element rule on a tile that is not tile_full, with ps = min(S, prefix) and ws = min(S, window)
// precomputed.  For a query row q < S it equals retained(q, key, S, m): key <= q implies
// key < S, and key + ws > q is key >= q - ws + 1.
__host__ __device__ inline bool keep_key(int q, int key, int ps, int ws, int kind) {
  return key <= q && (kind == 0 || key < ps || key >= q - ws + 1);
}

// The compares the attention kernel applies to a tile that is not tile_full for the wavefront
// rows [wq0, wq1] (wq0 <= wq1 < S): the tile's position decides which conjuncts of keep_key can
// fail for those rows, so most boundary tiles need one compare per key.
enum TileMaskCase {
  kDropAbove = 0,         // every key in the prefix or in every row's window: drop key > q
  kDropBeforeWindow = 1,  // past the prefix, left of every row: drop key < q - ws + 1
  kDropPastPrefix = 2,    // left of every row's window (the prefix's partial tile): drop key >= ps
  kDropGeneral = 3        // straddles the prefix end and a window start: the full rule
};
__host__ __device__ inline int tile_mask_case(int kb, int wq0, int wq1, int ps, int ws, int kind) {
  const int ke = kb + kTileK - 1;
  if (kind == 0 || ke < ps || kb >= wq1 - ws + 1) return kDropAbove;
  if (kb >= ps && ke <= wq0) return kDropBeforeWindow;
  if (ke < wq0 - ws + 1) return kDropPastPrefix;
  return kDropGeneral;
}
// The rule of each case for key `key` of row q -- what the kernel's compares keep.
__host__ __device__ inline bool tile_case_keeps(int c, int q, int key, int ps, int ws) {
  switch (c) {
    case kDropAbove: return key <= q;
    case kDropBeforeWindow: return key >= q - ws + 1;
    case kDropPastPrefix: return key < ps;
    default: return !(key > q || (key >= ps && key < q - ws + 1));
  }
}

// Keys the attention kernel keeps for query row q of a sequence of length S, as a bitmask row
// (word k/32, bit k%32; `row` pre-zeroed, `words` = ceil(S/32)).  Walks the kernel's own
// iteration with the kernel's own per-tile decisions: every wavefront of a work item visits the
// work item's tile ranges (key_tiles over its 64 rows); a tile that is tile_full for the
// wavefront's 32 rows keeps all its keys, any other tile keeps what its tile_mask_case rule keeps.
__host__ __device__ inline void kept_keys_row(int q, int S, const MaskSpec& m, uint32_t* row,
                                              int words) {
  const int blk_q0 = (q / kBlockQ) * kBlockQ;
  const int blk_q1 = (S < blk_q0 + kBlockQ ? S : blk_q0 + kBlockQ) - 1;
  const int wq0 = (q / kWaveQ) * kWaveQ;
  const int wq1 = (S - 1 < wq0 + kWaveQ - 1) ? S - 1 : wq0 + kWaveQ - 1;
  const int ps = S < m.prefix ? S : m.prefix;
  const int ws = S < m.window ? S : m.window;
  const TileRanges tiles = key_tiles(blk_q0, blk_q1, S, m);
  for (int it = 0; it < tiles.count(); ++it) {
    const int kb = tiles.at(it) * kTileK;
    const bool full = tile_full(kb, wq0, wq1, S, m);
    const int c = tile_mask_case(kb, wq0, wq1, ps, ws, m.kind);
    for (int wd = 0; wd < kTileK / 32; ++wd) {
      uint32_t word = 0;
      for (int b = 0; b < 32; ++b) {
        const int key = kb + 32 * wd + b;
        if (full || tile_case_keeps(c, q, key, ps, ws)) word |= 1u << b;
      }
      const int wi = kb / 32 + wd;
      if (wi < words) row[wi] = word;
    }
  }
}

// One work entry of a launch: key tiles [tile_begin, tile_end) of the key_tiles() list of the
// item (sequence start token, length, query block, sequence<<4 | kv_head).  An item whose tiles
// are spread over several entries ("chunks") has split >= 0: its chunks share counter `split`,
// and part = ci | nchunks << 4 | first_partial << 8 (chunk ci of nchunks, whose partial
// results sit at workspace index first_partial + ci).  Unsplit items have split = -1, part = 0.
struct WorkItem {
  int seq_start;
  int seq_len;
  int q_block;
  int seq_kvh;
  int tile_begin;
  int tile_end;
  int split;
  int part;
};
constexpr int kMaxChunks = 8;  // chunks per split item (the merge kernel takes up to 8 per pass)

typedef _Float16 half_t;

// Arguments of one attention launch (host planner -> kernels).
struct AttnParams {
  const half_t* q;
  const half_t* k;
  const half_t* v;  // already offset by v_offset
  half_t* o;
  half_t* o_last;
  uint32_t q_stride_b, k_stride_b, v_stride_b, o_stride_b;  // row strides in bytes (< 2^31)
  const WorkItem* work;       // work items grouped by slot
  const int32_t* slot_begin;  // slot b owns work[slot_begin[b] .. slot_begin[b+1])
  int32_t n_slots;            // workgroups launched
  MaskSpec mask;
  float scale_log2;           // (1/sqrt(128)) * log2(e)
  float* partials;            // split chunks' partial results (one record set per chunk)
  const WorkItem* splits;     // chunk 0 of each split item, for the merge kernel
  int32_t n_splits;
  // Mask check only (qattn_debug_run_mask): when non-NULL the kernel also writes, for every
  // query head h, packed row t and key k of t's sequence, bit k%32 of word
  // maskbits[(h * mask_rows + t) * mask_words + k/32] iff the masked score it computed for
  // (t, k) is finite, i.e. the key survived the compares it executed.
  uint32_t* maskbits;
  int32_t mask_rows;   // packed tokens T
  int32_t mask_words;  // words per row: ceil(longest sequence / 32)
  // Phase timeline only (qattn_debug_run_timeline): when non-NULL the kernel also writes
  // kTimelineStamps s_memrealtime values (100 MHz) per workgroup b at timeline[b * kTimelineStamps]:
  // 0 start, 1 first loads landed, per entry e < 15 at 2 + 8 e: +0 entry top, +1 after its first
  // tile's barrier, +2 after its last tile's barrier, +3 after that tile issued the next
  // entry's loads, +4 after its last PV, +5 after the hand-over wait, +6 after the rows were
  // staged (or the partials stored) and the next S(0) issued, +7 after the row stores
  // (entries past 14 share entry 14's stamps), kTimelineStamps - 1 end.  Unreached stamps stay 0.
  uint32_t* timeline;
};
constexpr int kTimelineStamps = 128;

}  // namespace qattn
