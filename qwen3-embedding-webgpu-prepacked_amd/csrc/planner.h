// planner.h -- host planner of the attention operator: a validated run description (cu_seqlens,
// mask) -> work entries of (sequence, KV head, 64-query block, key-tile range) grouped into the
// persistent workgroups ("slots") of one launch, plus the launch arguments.
//
// Replaces CausalAttentionKernel.createRun (src/webgpu/ops.ts:327-343): the reference bakes
// [batch, sequence, heads, value_stride, value_offset] into a uniform buffer and dispatches
// ceil(S/16) x batch*16 workgroups over a padded batch.  Here the work list is built from
// cu_seqlens: no padded rows, both heads of a GQA group per entry, heaviest entries first so the
// longest causal rows start early, and one launch per layer regardless of sequence length (the
// reference switches to a chunked two-pass path above 8192 tokens, ops.ts:328-342).
#pragma once
#include <stdint.h>

#include <vector>

#include "../../include/qattn.h"
#include "attn_common.h"

namespace qattn {

// Slots: persistent workgroups of one launch.  Two fit on a CU (64 KiB LDS, <= 256 VGPRs each);
// workgroup b is dispatched to XCD b % kXcds, so the planner puts every item of KV head g on
// slots b = kXcds * j + g % kXcds and that head's K/V tiles stay in one XCD's L2.
constexpr int kXcds = 8;
constexpr int kBlocksPerCU = 2;
constexpr int kDefaultSlots = 256 * kBlocksPerCU;  // MI355X: 256 CUs
// Partial result of one chunk: per wavefront (4) and lane (64), the lane's 64 O^T values of its
// row divided by the row sum, as fp16 (32 words), then m and l (log2-domain row max, row sum)
// and two pad words.
constexpr int kPartialFloats = 36;
constexpr size_t kPartialBytes = (size_t)kWaves * 64 * kPartialFloats * 4;

struct Plan {
  std::vector<WorkItem> items;       // grouped by slot, heaviest first within a slot
  std::vector<int32_t> slot_begin;   // n_slots + 1 offsets into items
  std::vector<WorkItem> split_heads; // chunk 0 of each split item, by split id
  int32_t splits = 0;                // items spread over several chunks
  int32_t partials = 0;              // chunk partial-result records the workspace holds
};

// Closed form of the retained-pair count of one sequence (sum over q of |{k : retained(q,k)}|).
int64_t pairs_of(int64_t L, const MaskSpec& m);

// Plans a description that validate_desc accepted: entries for at most max_slots workgroups
// (rounded up to one per XCD), the run figures and the mask the kernel applies.
void plan_work(const qattn_run_desc* d, int max_slots, Plan* out, qattn_run_info* info_out,
               MaskSpec* mask_out);

// Launch arguments of a validated description whose work list sits at `plan` (entries, then the
// split items' chunk-0 entries, then the slot offsets).
void fill_params(AttnParams* p, const qattn_run_desc* d, const MaskSpec& mask, int32_t slots,
                 const void* plan, size_t items_bytes, size_t heads_bytes);

}  // namespace qattn
