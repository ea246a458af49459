// attn_fwd.hip -- causal / prefix+local GQA prefill attention for gfx950 (MI355X).
//
// Replaces the reference's tiled flash attention shader (src/webgpu/ops.ts:168-241).  Same
// result (softmax(mask(QK^T)/sqrt(128)) V per query head, mask ops.ts:205-209,220), computed
// the CDNA4 way:
//   * a work item = (sequence, KV head, 64 query positions) and BOTH query heads of the GQA
//     group (4 wavefronts x 32 rows), so each K/V tile is staged in LDS once for two heads;
//   * persistent workgroups: the host planner gives every workgroup ("slot") a list of work
//     items, balanced longest-first, and keeps each KV head's items on one XCD (slot b runs on
//     XCD b % 8) so that head's K/V stays in one L2.  While an item runs its last key tile, the
//     workgroup already loads the next item's Q and first two K tiles, and it never waits for
//     an item's O stores: loads, MFMA work and stores of neighbouring items overlap;
//   * S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_32x32x16_f16 (fp16 in, fp32 accumulate), so
//     every lane owns one query row: the row max / row sum need one permlane32 swap;
//   * K/V tiles go HBM -> LDS with buffer_load ... lds (no staging registers); the buffer
//     resource spans only the sequence's rows, so keys past its end arrive as zeros;
//   * LDS tiles are row-major 256 B rows with a 16 B-granular XOR swizzle chosen so that the K
//     fragment reads (ds_read_b128) and the V^T fragment reads (ds_read_b64_tr_b16, the gfx950
//     LDS transpose load) are bank-conflict free;
//   * software pipelined: iteration j issues the S^T MFMAs of tile j+1 and the PV MFMAs of tile
//     j-1 in the same basic block as the softmax VALU work of tile j; the score / probability
//     registers alternate between two sets by iteration parity (no copies); K and V are double
//     buffered in LDS;
//   * no per-tile row max: probabilities are taken against the entry's first-tile row max and
//     O and l are rescaled only when a later tile's probabilities could leave fp16 range;
//   * causal and prefix/local masks skip whole key tiles (key_tiles); element masks run only on
//     tiles that straddle a boundary (tile_full);
//   * output rows go through LDS and leave as whole 128-byte lines, non-temporal, so the L2
//     keeps the K/V tiles that later items of the same sequence re-read.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "attn_common.h"

namespace qattn {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) s4 lds_s4_t;

constexpr int kRowBytes = kHeadDim * 2;                      // 256 B per key row in LDS
constexpr int kTileBytes = kTileK * kRowBytes;               // 16 KiB per K or V tile
constexpr int kLoadsPerTile = kTileBytes / (kThreads * 16);  // 16 B per lane per load: 4
constexpr float kLazyLimit = 32768.f;


// Partial result of one chunk of a split item, per wavefront: 9 records of 64 lanes x 16 bytes
// (record 2 db + h: the lane's O^T accumulators o[db][8h .. 8h+7] divided by the row's sum, as
// fp16; record 8: m, the row's sum l, 0, 0 in fp32), so every access is a coalesced 1 KiB row.
// fp16 is the output's own precision: the merge adds at most one more fp16 rounding per chunk.
constexpr int kPartialRecords = 9;

// Vector-memory instructions per lane that one item's prologue loads (Q: 8 x 16 B, K tiles 0
// and 1: kLoadsPerTile each) and that one item's epilogue stores (O rows, 8 x 16 B per lane, plus
// as many for the o_last row when the run has one; always issued: out-of-range rows are dropped
// by the buffer resource).  The s_waitcnt counts below rely on these being exact; vector memory
// operations retire in issue order.
constexpr int kPrefetchOps = 8 + 2 * kLoadsPerTile;
template <bool LAST>
constexpr int kStoreOps = LAST ? 16 : 8;

// s_waitcnt vmcnt(N) only (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ inline void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

__device__ inline f16x mfma32(h8 a, h8 b, f16x c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Raw buffer resource over `bytes` bytes at `base`; loads past the end return zeros and stores
// past the end are dropped.
__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// x combined with the other half-wave's x (lane l <-> lane l^32).
__device__ inline float pair_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float pair_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Offset of S^T accumulator element r (0..31 over the two 32-key blocks) from kb + 4*hl.
__device__ constexpr int key_off(int r) { return 32 * (r >> 4) + 8 * ((r & 15) >> 2) + (r & 3); }

__device__ inline uint32_t pack2(float a, float b) {
  const h2 v = {(half_t)a, (half_t)b};
  return __builtin_bit_cast(uint32_t, v);
}

// The low / high fp16 of a dword, widened (integer extraction, not a vector element).
__device__ inline float half_lo(uint32_t d) { return (float)__builtin_bit_cast(half_t, (unsigned short)(d & 0xFFFFu)); }
__device__ inline float half_hi(uint32_t d) { return (float)__builtin_bit_cast(half_t, (unsigned short)(d >> 16)); }

// Record 0 of partial result `index` for (wave, lane); record r is 64 float4 further per r.
__device__ inline float __attribute__((ext_vector_type(4)))* partial_records(float* partials, int index,
                                                                               int wave, int lane) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  return reinterpret_cast<f4*>(partials) + ((size_t)index * kWaves + wave) * kPartialRecords * 64 + lane;
}

// Output rows of one wavefront, staged through LDS.  O = O^T / l for query rows q_row0 ..
// q_row0 + 31 (lanes l and l^32 hold row q_row0 + l % 32, dims 32db + 8g + 4hl + 0..3); one
// permlane32 swap per dword leaves each lane 8 consecutive dims (16 B): g = 2gp in the low
// half-wave, g = 2gp+1 in the high one.  stage_rows writes the 32 fp16 rows into 8 KiB of a free
// V buffer (row-major 256 B rows, 16 B chunk c of row r at c ^ (r & 15): conflict-free both
// ways); flush_rows reads them back four whole rows per instruction and stores them into O and
// (for the sequence's last row) o_last, so every store writes whole cache lines instead of 32 B
// pieces of 32 rows.  Exactly kStoreOps<LAST> buffer stores per lane; rows past the sequence (and
// every row but the last, for o_last) get an offset beyond the buffer resource, so their stores
// are dropped (S * o stride < 2^31 is validated on the host).  The stores are non-temporal (the
// output is not read again by this launch), which keeps L2 for the K/V tiles: with whole-line
// stores that measured 16x500 -5.8%, 1x5000 -2%, 1x1500 -3.4% (with the earlier 32 B pieces,
// non-temporal stores were 10-40% slower).
constexpr int kNonTemporal = 2;  // buffer instruction cache-policy operand: nt
typedef __attribute__((address_space(3))) char lds_char_t;
typedef uint32_t u4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) u4 lds_u4_t;
__device__ inline lds_char_t* row_stage(lds_char_t* v0, lds_char_t* v1) {
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  return (wave < 2 ? v0 : v1) + (wave & 1) * (kWaveQ * kRowBytes);
}
__device__ inline void stage_rows(const f16x (&o)[4], float l_run, lds_char_t* stage) {
  int lane = threadIdx.x & 63;
  asm volatile("" : "+v"(lane));  // the LDS addresses below are computed here, not hoisted
  const int lq = lane & 31, hl = lane >> 5;
  const float l_tot = pair_sum(l_run);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int gp = 0; gp < 2; ++gp) {
      const f16x& v = o[db];
      const int ga = 4 * (2 * gp), gb = 4 * (2 * gp + 1);
      const uint32_t a0 = pack2(v[ga] * inv, v[ga + 1] * inv), a1 = pack2(v[ga + 2] * inv, v[ga + 3] * inv);
      const uint32_t b0 = pack2(v[gb] * inv, v[gb + 1] * inv), b1 = pack2(v[gb + 2] * inv, v[gb + 3] * inv);
      const auto r0 = __builtin_amdgcn_permlane32_swap(a0, b0, false, false);
      const auto r1 = __builtin_amdgcn_permlane32_swap(a1, b1, false, false);
      const int cw = 4 * db + 2 * gp + hl;  // 16 B chunk of row lq
      *(lds_u4_t*)(stage + lq * kRowBytes + ((cw ^ (lq & 15)) << 4)) = u4{r0[0], r1[0], r0[1], r1[1]};
    }
}
template <bool LAST>
__device__ inline void flush_rows(const AttnParams& p, int seq_start, int S, int seq, int head, int q_row0,
                                  const lds_char_t* stage) {
  int lane = threadIdx.x & 63;
  asm volatile("" : "+v"(lane));
  const uint32_t ostride_b = p.o_stride_b;
  const auto ors = make_rsrc(reinterpret_cast<const char*>(p.o) + (uint64_t)seq_start * ostride_b + head * kRowBytes,
                             (uint32_t)S * ostride_b);
  const auto lrs = make_rsrc(p.o_last + (int64_t)seq * (kQHeads * kHeadDim) + head * kHeadDim,
                             p.o_last ? kRowBytes : 0u);
#pragma unroll
  for (int j = 0; j < kWaveQ / 4; ++j) {
    const int row = 4 * j + (lane >> 4), cr = lane & 15, q = q_row0 + row;
    const u4 val = *(const lds_u4_t*)(stage + row * kRowBytes + ((cr ^ (row & 15)) << 4));
    if (LAST)
      __builtin_amdgcn_raw_buffer_store_b128(val, lrs, (q == S - 1 ? 0u : 0x80000000u) + 16u * cr, 0, kNonTemporal);
    __builtin_amdgcn_raw_buffer_store_b128(val, ors, (q < S ? (uint32_t)q * ostride_b : 0x80000000u) + 16u * cr, 0,
                                           kNonTemporal);
  }
}

// SPLIT: the plan has split items (partial-result path compiled in).  LAST: the run writes
// o_last rows.  MASKBITS: also report the kept keys (p.maskbits; the mask check only).
// TIMELINE: also record each workgroup's phase timestamps (p.timeline; qattn_debug_run_timeline).
template <bool SPLIT, bool LAST, bool MASKBITS = false, bool TIMELINE = false>
__global__ __launch_bounds__(kThreads, 2) void attn_fwd_kernel(AttnParams p) {
  // K and V tiles, double buffered, 16 KiB each.  Four distinct objects (not offsets into one
  // array) with buffer choices fixed at compile time, so the compiler can see that the LDS-DMA
  // loads in flight never alias the tile being read and does not wait for them.
  __shared__ __attribute__((aligned(1024))) char sK0[kTileBytes];
  __shared__ __attribute__((aligned(1024))) char sK1[kTileBytes];
  __shared__ __attribute__((aligned(1024))) char sV0[kTileBytes];
  __shared__ __attribute__((aligned(1024))) char sV1[kTileBytes];

  // The work list is read-only for the whole launch: read it through the constant address
  // space so item loads are scalar loads, which no vector-memory wait (for the O stores) covers.
  typedef __attribute__((address_space(4))) const int32_t const_i32_t;
  const_i32_t* const work_words = (const_i32_t*)p.work;
  auto work = [&](int i) {
    const_i32_t* w = work_words + 8 * i;
    return WorkItem{w[0], w[1], w[2], w[3], w[4], w[5], w[6], w[7]};
  };
  const int i_begin = ((const_i32_t*)p.slot_begin)[blockIdx.x];
  const int i_end = ((const_i32_t*)p.slot_begin)[blockIdx.x + 1];
  if (i_begin >= i_end) return;

  // Phase timestamps (TIMELINE only): s_memrealtime (100 MHz) read by thread 0 into LDS at
  // kTimelineStamps fixed points, written out once the workgroup is done (LDS, so the vector-
  // memory counts that the waits rely on are unchanged).
  __shared__ uint32_t tl_stamps[TIMELINE ? kTimelineStamps : 1];
  auto stamp = [&](int i) {
    if constexpr (TIMELINE) {
      if (threadIdx.x == 0) tl_stamps[i] = (uint32_t)__builtin_amdgcn_s_memrealtime();
    }
  };
  if constexpr (TIMELINE) {
    if (threadIdx.x < kTimelineStamps) tl_stamps[threadIdx.x] = 0;
  }
  stamp(0);
  int tl_entry = 2;  // first stamp of the current entry: 2 + 8 min(entry, 14)

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: keeps rsrc/M0 in SGPRs
  const int lane = tid & 63;
  const int lq = lane & 31;  // query row of this lane inside the wave's 32-row tile
  const int hl = lane >> 5;  // which half of the MFMA K dimension this lane feeds
  const int head_in_group = wave >> 1;
  const int wave_q = (wave & 1) * kWaveQ;
  const MaskSpec mask = p.mask;
  const float c = p.scale_log2;
  const uint32_t qstride_b = p.q_stride_b, kstride_b = p.k_stride_b, vstride_b = p.v_stride_b;

  // ---- tile loads: kLoadsPerTile buffer_load...lds per lane per tile; instruction j of wave
  // `wave` fills LDS rows 16j + 4*wave .. +3 (1 KiB, lane-contiguous).  Lane writes physical chunk
  // lane&15 of row r with the logical 16 B chunk (lane&15) ^ swizzle(r) of key row kb + r.
  // Row r = 16j + r0 with r0 = 4*wave + lane/16, so r & 15 = r0: the swizzle is the same for
  // every j and instruction j only adds 16j rows.  That step goes into the VGPR offset (one add),
  // not the SGPR offset, because the buffer range check that zero-fills rows past the sequence
  // covers the VGPR and immediate offsets only.
  const int r0 = 4 * wave + (lane >> 4), pc = lane & 15;
  const uint32_t koff = (uint32_t)r0 * kstride_b + (uint32_t)((pc ^ r0) << 4);
  const uint32_t voff = (uint32_t)r0 * vstride_b + (uint32_t)((pc ^ ((r0 & 3) << 2)) << 4);
  // Key tile `kt` of a sequence of S rows starting at `base` (kt * kTileK < S, or S = 0 for an
  // empty range).
  auto tile_rsrc = [&](const char* base, uint32_t stride_b, int kt, int S) {
    const int kb = kt * kTileK;
    return make_rsrc(base + (int64_t)kb * stride_b, S > kb ? (uint32_t)(S - kb) * stride_b : 0u);
  };
  auto load_part = [&](char* dst, __amdgpu_buffer_rsrc_t rs, uint32_t stride_b, uint32_t off, int j) {
    // The add stays here (not hoisted into four loop-invariant registers).
    uint32_t step = (uint32_t)(16 * j) * stride_b;
    asm volatile("" : "+s"(step));
    // The destination (M0) is formed here from one per-wave offset, not kept in 16 registers.
    uint32_t wbase = (uint32_t)wave * 1024u;
    asm volatile("" : "+s"(wbase));
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(dst + j * 4096 + wbase), 16, off + step, 0, 0, 0);
  };
  auto load_tile = [&](char* dst, const char* base, uint32_t stride_b, uint32_t off, int kt, int S) {
    const auto rs = tile_rsrc(base, stride_b, kt, S);
#pragma unroll
    for (int j = 0; j < kLoadsPerTile; ++j) load_part(dst, rs, stride_b, off, j);
  };

  // ---- LDS read addresses.
  // K (A operand of S^T): lane reads key row lq (+32 for the second block), logical chunk
  // 2*st + hl, stored at physical chunk (2*st + hl) ^ (lq & 15).  Bit 0 of that chunk is
  // hl ^ lq, bits 3:1 are st ^ ((lq & 15) >> 1), so the byte address is
  // kread_base + ((st << 5) ^ kread_xor): one v_xad_u32 per step instead of 8 live registers.
  const uint32_t kread_base = lq * kRowBytes + (((hl ^ lq) & 1) << 4);
  const uint32_t kread_xor = ((lq & 15) >> 1) << 5;
  // V^T (A operand of O^T = V^T P^T) through ds_read_b64_tr_b16: in each 16-lane group G the
  // source lane a reads 4 halves at key row 4*(G>>1) + (a>>2) (+16t, +8 for slots 4..7), dims
  // 32db + 16(G&1) + 4(a&3); lane a then receives V[4 keys][dim 32db + 16(G&1) + a].  V rows are
  // stored with physical chunk = logical chunk ^ ((row & 3) << 2): the 32 lanes the LDS serves
  // per pass read rows 4i..4i+3 x the 4 chunks of dims 32db..32db+31, and the swizzle spreads
  // them over all 16 chunks = all 64 banks.
  uint32_t vread[4];
  {
    const int a = lane & 15, G = lane >> 4;
    const int row = 4 * (G >> 1) + (a >> 2);
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const int chunk = (4 * db + 2 * (G & 1) + ((a & 3) >> 1)) ^ ((a >> 2) << 2);
      vread[db] = row * kRowBytes + (chunk << 4) + ((a & 1) << 3);
    }
  }

  // ---- Q fragment (B operand of S^T = K Q^T): lane = query row, 8 consecutive dims per step.
  h8 qreg[8];

  // The loads that start a work item: this wave's Q rows into qreg, K tiles 0 and 1 into sK0 /
  // sK1 (tile 0 twice for a one-tile item, so the instruction count never varies).  Exactly
  // kPrefetchOps vector-memory instructions per lane; with real = false every buffer range is
  // empty (the instructions read nothing and write zeros).
  auto start_loads = [&](const WorkItem& w, bool real) {
    const int S = w.seq_len, kvh = w.seq_kvh & 15, q0 = w.q_block * kBlockQ;
    const TileRanges t = key_tiles(q0, min(S, q0 + kBlockQ) - 1, S, mask);
    const int tb = w.tile_begin, t1 = w.tile_end - w.tile_begin > 1 ? tb + 1 : tb;
    const char* qhead = reinterpret_cast<const char*>(p.q) + (uint64_t)w.seq_start * qstride_b +
                        (kvh * kGroup + head_in_group) * kRowBytes;
    const auto rs = make_rsrc(qhead, real ? (uint32_t)S * qstride_b : 0u);
    const uint32_t row_off = (uint32_t)(q0 + wave_q + lq) * qstride_b + 16u * hl;
#pragma unroll
    for (int st = 0; st < 8; ++st)
      qreg[st] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(rs, row_off + 32u * st, 0, 0));
    const char* kb = reinterpret_cast<const char*>(p.k) + (uint64_t)w.seq_start * kstride_b + kvh * kRowBytes;
    load_tile(sK0, kb, kstride_b, koff, t.at(tb), real ? S : 0);
    load_tile(sK1, kb, kstride_b, koff, t.at(t1), real ? S : 0);
  };

  // ---- per-entry state (uniform over the workgroup except q_pos).  Local tile it is key tile
  // tiles.at(t0 + it) of the item; an unsplit entry has t0 = 0 and ntiles = tiles.count().
  bool has_next = false;
  int seq_start = 0, S = 1, kvh = 0, seq = 0, wq0 = 0, wq1 = 0, q_pos = 0, ps = 0, ws = 0, ntiles = 0, t0 = 0;
  TileRanges tiles{};
  const char* kbase = nullptr;
  const char* vbase = nullptr;

  // S^T (64 keys x 32 queries) for the K tile in `kt`.  Lane holds S^T[key][q_pos] for
  // key = kb + 4*hl + key_off(r), r = 0..31 over (s[0], s[1]).
  // `step_hook(st)` runs after step st's MFMAs (the main loop issues its tile loads there, one
  // per step, so they reach the texture unit spread out instead of in one burst per iteration).
  // Each step's K fragments are read one step ahead, before the previous step's tile load (which
  // the compiler may not move LDS reads across), so no MFMA waits for its own LDS read.
  auto qk = [&](const char* kt, f16x (&s)[2], auto step_hook) {
    uint32_t kx = kread_xor;
    asm volatile("" : "+v"(kx));  // keeps the 8 addresses from being hoisted into registers
    auto frag = [&](int st, int half) {
      const uint32_t ka = kread_base + (((uint32_t)st << 5) ^ kx) + half * 32 * kRowBytes;
      return *reinterpret_cast<const h8*>(kt + ka);
    };
    h8 a0 = frag(0, 0), a1 = frag(0, 1);
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      h8 n0 = a0, n1 = a1;
      if (st < 7) {
        n0 = frag(st + 1, 0);
        n1 = frag(st + 1, 1);
      }
      // step 0 accumulates onto the inline constant 0 (no zeroed registers)
      s[0] = mfma32(a0, qreg[st], st == 0 ? f16x{} : s[0]);
      s[1] = mfma32(a1, qreg[st], st == 0 ? f16x{} : s[1]);
      step_hook(st);
      a0 = n0;
      a1 = n1;
    }
  };
  auto no_hook = [](int) {};

  // O^T (128 d x 32 q) += V^T (128 x 64 keys) . P^T.  Step t covers keys kb+16t..kb+16t+15;
  // slot j of lane half hl is key 16t + 8*(j>>2) + 4*hl + (j&3), whose probability is pf[t][j].
  f16x o[4];
  auto pv = [&](const char* vt, const h8 (&pf)[4]) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const char* vp = vt + vread[db] + t * 4096;
        const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4_t*)vp);
        const s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4_t*)(vp + 2048));
        const h4 lo_h = __builtin_bit_cast(h4, lo), hi_h = __builtin_bit_cast(h4, hi);
        const h8 va = {lo_h[0], lo_h[1], lo_h[2], lo_h[3], hi_h[0], hi_h[1], hi_h[2], hi_h[3]};
        o[db] = mfma32(va, pf[t], o[db]);
      }
    }
  };

  // Element mask of a boundary tile: the keys its tile_mask_case rule drops become -inf.  With
  // o = key_off(r) = key - kl (kl = kb + 4 hl), the rules are compares of compile-time offsets
  // against per-lane thresholds (d1 = q_pos - kl, pe = ps - kl, d2 = d1 - ws + 1):
  //   kDropAbove        drop o > d1                     (key > q)
  //   kDropBeforeWindow drop o < d2                     (key < q - ws + 1)
  //   kDropPastPrefix   drop o >= pe                    (key >= ps)
  //   kDropGeneral      drop o > d1 || (o >= pe && o < d2)
  // The case is uniform over the wavefront, so most boundary tiles cost one compare + one select
  // per element.  kept_keys_row() (attn_common.h) evaluates the same cases on the host.
  auto apply_mask = [&](f16x (&s)[2], int kb) {
    const int kl = kb + 4 * hl;
    const int d1 = q_pos - kl;
    auto drop_if = [&](auto pred) {
#pragma unroll
      for (int r = 0; r < 32; ++r) s[r >> 4][r & 15] = pred(key_off(r)) ? -INFINITY : s[r >> 4][r & 15];
    };
    switch (tile_mask_case(kb, wq0, wq1, ps, ws, mask.kind)) {
      case kDropAbove:
        drop_if([&](int o) { return o > d1; });
        break;
      case kDropBeforeWindow: {
        const int d2 = d1 - ws + 1;
        drop_if([&](int o) { return o < d2; });
        break;
      }
      case kDropPastPrefix: {
        const int pe = ps - kl;
        drop_if([&](int o) { return o >= pe; });
        break;
      }
      default: {
        const int pe = ps - kl, d2 = d1 - ws + 1;
        // bitwise, not short-circuit: one select per element instead of a branch
        drop_if([&](int o) { return (o > d1) | ((o >= pe) & (o < d2)); });
      }
    }
  };

  // Mask check: which keys of this tile survived for this lane's row (finite masked score).
  // Lane half hl holds keys kb + 4hl + key_off(r); one permlane32 swap merges the two halves,
  // leaving the word of keys kb..kb+31 in the low half-wave and kb+32..kb+63 in the high one.
  // (Extra stores: the pipeline's vmcnt waits only become stricter.)
  auto record_mask = [&](const f16x (&s)[2], int kb) {
    uint32_t w0 = 0, w1 = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int bit = 8 * (r >> 2) + (r & 3) + 4 * hl;
      w0 |= (s[0][r] != -INFINITY ? 1u : 0u) << bit;
      w1 |= (s[1][r] != -INFINITY ? 1u : 0u) << bit;
    }
    const auto x = __builtin_amdgcn_permlane32_swap(w0, w1, false, false);
    const int word = kb / 32 + hl;
    if (q_pos < S && word < (S + 31) / 32) {
      const int head = kvh * kGroup + head_in_group;
      p.maskbits[((size_t)head * p.mask_rows + seq_start + q_pos) * p.mask_words + word] = x[0] | x[1];
    }
  };

  // Online softmax.  The probabilities of a row are taken against a reference m_run (log2
  // domain): P = f16(2^(s c - m_run)), O = sum P V, l = sum P.  m_run is the row max of the
  // entry's first tile and moves only when a later tile's probabilities could leave fp16 range:
  // no per-tile max, no per-tile rescale.  A lane whose half-row sum of one tile exceeds
  // kLazyLimit (2^15; each P is then <= 2^15 < 65504, the fp16 maximum) -- or is inf / NaN
  // (m_run still -inf: every key so far masked) -- sends the wavefront through the full update:
  // tile max, new reference, O and l scaled by alpha, P recomputed.  After the first tile with
  // a key, l >= 1 (the max key has P = 1), so small P values lose nothing relative to l.
  float m_run = -INFINITY;  // reference (log2 domain) the probabilities are taken against
  float l_run = 0.f;        // running sum of the fp16-rounded probabilities
  // P in fp16 feeds the PV MFMA; the row sum adds those same rounded values (exactly: each f16
  // is widened inside v_fma_mix_f32), so O is an exact weighted mean of V and the fp16 rounding
  // of P only perturbs the weights.
  auto probs = [&](const f16x (&s)[2], h8 (&pf)[4], float m_use) {
    float ps0 = 0.f, ps1 = 0.f;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int r = 8 * t + j;
        pf[t][j] = (half_t)__builtin_amdgcn_exp2f(fmaf(s[r >> 4][r & 15], c, -m_use));
      }
      typedef uint32_t u4 __attribute__((ext_vector_type(4)));
      const u4 pairs = __builtin_bit_cast(u4, pf[t]);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float& ps = (j & 1) ? ps1 : ps0;
        asm("v_fma_mix_f32 %0, %1, 1.0, %0 op_sel_hi:[1,0,0]\n\t"
            "v_fma_mix_f32 %0, %1, 1.0, %0 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
            : "+v"(ps)
            : "v"(pairs[j]));
      }
    }
    return ps0 + ps1;
  };
  auto tile_max = [&](const f16x (&s)[2]) {
    float mx = fmaxf(fmaxf(s[0][0], s[0][1]), s[0][2]);
#pragma unroll
    for (int r = 3; r < 31; r += 2) mx = fmaxf(fmaxf(mx, s[r >> 4][r & 15]), s[(r + 1) >> 4][(r + 1) & 15]);
    mx = fmaxf(mx, s[1][15]);
    return pair_max(mx);
  };
  // The entry's first tile: O = 0, l = 0; the reference is this tile's row max.
  auto softmax_first = [&](const f16x (&s)[2], h8 (&pf)[4]) {
    m_run = tile_max(s) * c;
    l_run = probs(s, pf, m_run == -INFINITY ? 0.f : m_run);
  };
  // Later tiles: the fast path, or the full update for the whole wavefront when any lane needs it.
  auto softmax_next = [&](const f16x (&s)[2], h8 (&pf)[4]) {
    float psum = probs(s, pf, m_run);
    if (__builtin_amdgcn_ballot_w64(!(psum <= kLazyLimit)) != 0) {
      const float m_new = fmaxf(m_run, tile_max(s) * c);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);  // 0 while m_run is -inf
      psum = probs(s, pf, m_use);
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db] *= alpha;
      l_run *= alpha;
      m_run = m_new;
    }
    l_run += psum;
  };

  // Two register sets for scores / probabilities, alternating by iteration parity.
  f16x sA[2], sB[2];
  h8 pA[4], pB[4];

  // Iteration `it` of the current item, B = it & 1 (compile time).  Before it: S(it) in s_cur,
  // P(it-1) in p_prev, K(it+1) in sK<B^1>, V(it-1) in sV<B^1>.  It refills sK<B> with K(it+2) and
  // sV<B> with V(it), computes S(it+1) into s_nxt, adds P(it-1) V(it-1) to O and turns S(it)
  // into P(it) in p_cur.  The LAST iteration computes no S(it+1); it loads the next item's Q and
  // first K tiles instead (both K buffers and qreg are free by then).
  auto body = [&](auto bconst, int it, f16x (&s_cur)[2], f16x (&s_nxt)[2], h8 (&p_cur)[4],
                  const h8 (&p_prev)[4], bool with_pv, int next_index) {
    constexpr int B = decltype(bconst)::value;
    const bool last = it == ntiles - 1;
    char* const kfree = B == 0 ? sK0 : sK1;
    char* const knext = B == 0 ? sK1 : sK0;
    char* const vfree = B == 0 ? sV0 : sV1;
    char* const vprev = B == 0 ? sV1 : sV0;
    const int kb = tiles.at(t0 + it) * kTileK;
    // Loads issued last iteration have landed and every wavefront is done with last
    // iteration's reads of the buffers about to be refilled.  Iteration 0 issued nothing since
    // the item's start; only the previous item's O stores may still be in flight then.
    if (with_pv)
      __builtin_amdgcn_s_waitcnt(0);  // (gfx9 encoding 0: vmcnt/expcnt/lgkmcnt all zero)
    else
      wait_vmcnt<kStoreOps<LAST>>();
    __syncthreads();
    if (it == 0) stamp(tl_entry + 1);
    if (last) stamp(tl_entry + 2);
    // This iteration's tile loads: K(it+2) (if any) and V(it), one instruction per S(it+1) step
    // when there is one.
    const bool kload = it + 2 < ntiles;
    const auto krs = tile_rsrc(kbase, kstride_b, tiles.at(t0 + (kload ? it + 2 : it)), S);
    const auto vrs = tile_rsrc(vbase, vstride_b, tiles.at(t0 + it), S);
    if (last) {
      if (kload) load_tile(kfree, kbase, kstride_b, koff, tiles.at(t0 + it + 2), S);
      load_tile(vfree, vbase, vstride_b, voff, tiles.at(t0 + it), S);
    }
    // The slot's last item issues the same loads for its own Q / K(0) / K(1) as the "next"
    // item, over empty buffer ranges: they return zeros without touching memory (the re-read
    // of data long evicted from L2 was 13 MB of the 16x500 launch's HBM reads), and every path
    // issues the same vector-memory instruction count, so the waits below stay exact.
    if (last) start_loads(work(next_index), has_next);
    if (last) stamp(tl_entry + 3);
    if (!tile_full(kb, wq0, wq1, S, mask)) apply_mask(s_cur, kb);
    if constexpr (MASKBITS) record_mask(s_cur, kb);
    if (!last) {
      qk(knext, s_nxt, [&](int st) {
        if (st < kLoadsPerTile) {
          if (kload) load_part(kfree, krs, kstride_b, koff, st);
        } else {
          load_part(vfree, vrs, vstride_b, voff, st - kLoadsPerTile);
        }
      });
    } else {
      // No S(it+1) on the last tile.  Defining the set anyway (cheaply) keeps its previous
      // contents from staying live across the softmax.
      s_nxt[0] = f16x{};
      s_nxt[1] = f16x{};
    }
    if (with_pv) pv(vprev, p_prev);
    if (with_pv)
      softmax_next(s_cur, p_cur);
    else
      softmax_first(s_cur, p_cur);
    if (last) {
      // The item's last PV.  V(it) has landed once at most the next item's kPrefetchOps loads
      // are in flight.  (Here, not after the loop, so the V buffer stays a compile-time choice
      // and the compiler's own LDS-DMA wait can count the same way.)
      wait_vmcnt<kPrefetchOps>();
      __syncthreads();
      pv(vfree, p_cur);
      stamp(tl_entry + 4);
    }
  };

  // The item's last PV and its output rows.  O = O^T / l; lane pair (l, l^32) holds row q_pos,
  // dims 32db + 8g + 4hl + 0..3; one permlane32 swap per dword leaves each lane 8 consecutive
  // dims (16 B): g = 2gp in the low half-wave, g = 2gp+1 in the high one.
  // Chunk of a split item: store this chunk's partial softmax state (per lane: O / l, m, l) for
  // the merge kernel that runs after this launch; the chunk writes no output rows itself.
  // kPartialRecords vector stores; the next entry's first wait only ever waits for older ones.
  auto write_partial = [&](const WorkItem& w) {
    typedef float f4 __attribute__((ext_vector_type(4)));
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    const float l_tot = pair_sum(l_run);
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    f4* rec = partial_records(p.partials, (w.part >> 8) + (w.part & 15), wave, lane);
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int gh = 0; gh < 2; ++gh) {
        const f16x& v = o[db];
        const int b = 8 * gh;
        __builtin_nontemporal_store(
            u4{pack2(v[b] * inv, v[b + 1] * inv), pack2(v[b + 2] * inv, v[b + 3] * inv),
               pack2(v[b + 4] * inv, v[b + 5] * inv), pack2(v[b + 6] * inv, v[b + 7] * inv)},
            &reinterpret_cast<u4*>(rec)[64 * (2 * db + gh)]);  // whole 1 KiB rows, non-temporal
      }
    rec[64 * 8] = f4{m_run, l_tot, 0.f, 0.f};
  };

  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;

  start_loads(work(i_begin), true);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  stamp(1);
  qk(sK0, sA, no_hook);  // S(0) of the first entry
  for (int wi = i_begin; wi < i_end; ++wi) {
    const WorkItem cur = work(wi);
    tl_entry = 2 + 8 * min(wi - i_begin, 14);  // stamps 2 .. 121
    stamp(tl_entry);
    has_next = wi + 1 < i_end;
    const int next_index = has_next ? wi + 1 : wi;
    seq_start = cur.seq_start;
    S = cur.seq_len;
    kvh = cur.seq_kvh & 15;
    seq = cur.seq_kvh >> 4;
    const int blk_q0 = cur.q_block * kBlockQ;
    wq0 = blk_q0 + wave_q;
    wq1 = min(S - 1, wq0 + kWaveQ - 1);
    q_pos = wq0 + lq;
    ps = min(S, mask.prefix);
    ws = min(S, mask.window);
    tiles = key_tiles(blk_q0, min(S, blk_q0 + kBlockQ) - 1, S, mask);
    t0 = cur.tile_begin;
    ntiles = cur.tile_end - cur.tile_begin;
    kbase = reinterpret_cast<const char*>(p.k) + (uint64_t)seq_start * kstride_b + kvh * kRowBytes;
    vbase = reinterpret_cast<const char*>(p.v) + (uint64_t)seq_start * vstride_b + kvh * kRowBytes;
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db] = f16x{};
    m_run = -INFINITY;
    l_run = 0.f;

    // S(0) is in sA (computed before the loop or at the previous entry's end).
    body(I0{}, 0, sA, sB, pA, pB, false, next_index);
    for (int it = 1; it < ntiles; it += 2) {
      body(I1{}, it, sB, sA, pB, pA, true, next_index);
      if (it + 1 < ntiles) body(I0{}, it + 1, sA, sB, pA, pB, true, next_index);
    }
    // Hand-over: the next entry's Q, K(0), K(1) (issued with this entry's last tile) have landed
    // and every wave is past this entry's LDS reads, so the V buffers are free.  This entry's
    // output rows are normalised into them first, then the next S(0) goes to the matrix cores
    // (O and the next scores are never live together) and the rows are stored from LDS while
    // its MFMAs run.  The next entry's first barrier comes after these LDS reads; its first wait
    // allows for the stores still being in flight.
    if (wi + 1 < i_end) __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    stamp(tl_entry + 5);
    const bool rows = !SPLIT || cur.split < 0;
    lds_char_t* const stage = row_stage((lds_char_t*)sV0, (lds_char_t*)sV1);
    if (rows)
      stage_rows(o, l_run, stage);
    else
      write_partial(cur);
    if (wi + 1 < i_end) qk(sK0, sA, no_hook);
    stamp(tl_entry + 6);
    if (rows) flush_rows<LAST>(p, seq_start, S, seq, kvh * kGroup + head_in_group, wq0, stage);
    stamp(tl_entry + 7);
  }
  // The last item's unused prefetch (LDS-DMA included) lands before the workgroup leaves.
  __builtin_amdgcn_s_waitcnt(0);
  if constexpr (TIMELINE) {
    stamp(kTimelineStamps - 1);
    __syncthreads();
    if (threadIdx.x < kTimelineStamps) p.timeline[(size_t)blockIdx.x * kTimelineStamps + threadIdx.x] = tl_stamps[threadIdx.x];
  }
}

// Merge of split items (after attn_fwd_kernel, same stream).  Workgroup (split item i, wave w)
// redoes wavefront w's output rows of item i: thread 64 db + lane combines dims 32db..32db+31 of
// lane's row -- records 2db and 2db+1 of every chunk -- in chunk order: m = max_c m_c,
// w_c = 2^(m_c - m) l_c, O = sum_c w_c (O/l)_c / sum_c w_c (a chunk with no key for the row has
// m_c = -inf and weighs 0).  All of a thread's loads issue at once; stores go row-per-lane as the
// attention kernel's registers hold them, per 32-dim block.  The fp16 halves are taken apart with integer shifts: hipcc has compiled the
// element reads of a packed fp16 vector in an unrolled loop as element 0.
constexpr int kMergeMaxChunks = 8;  // chunks merged per pass (more are folded in further passes)
__global__ __launch_bounds__(kThreads) void attn_merge_kernel(AttnParams p) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(4))) const int32_t const_i32_t;
  const int item = blockIdx.x >> 2, wave = blockIdx.x & 3;
  const_i32_t* sw = (const_i32_t*)p.splits + 8 * item;
  const WorkItem w{sw[0], sw[1], sw[2], sw[3], sw[4], sw[5], sw[6], sw[7]};
  const int db = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, lq = lane & 31, hl = lane >> 5;
  const int nchunks = (w.part >> 4) & 15, first = w.part >> 8;
  float m = -INFINITY, l = 0.f;
  f4 acc[4] = {};
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
  for (int c0 = 0; c0 < nchunks; c0 += kMergeMaxChunks) {
    f4 ml[kMergeMaxChunks];
    u4 v[kMergeMaxChunks][2];
#pragma unroll
    for (int c = 0; c < kMergeMaxChunks; ++c) {
      if (c0 + c < nchunks) {
        const f4* rec = partial_records(p.partials, first + c0 + c, wave, lane);
        ml[c] = rec[64 * 8];
#pragma unroll
        for (int gh = 0; gh < 2; ++gh) v[c][gh] = reinterpret_cast<const u4*>(rec)[64 * (2 * db + gh)];
      }
    }
    float mp = m;
#pragma unroll
    for (int c = 0; c < kMergeMaxChunks; ++c)
      if (c0 + c < nchunks) mp = fmaxf(mp, ml[c][0]);
    const float rs = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - mp);  // rescale earlier passes
    l *= rs;
#pragma unroll
    for (int g = 0; g < 4; ++g) acc[g] *= rs;
#pragma unroll
    for (int c = 0; c < kMergeMaxChunks; ++c) {
      if (c0 + c < nchunks) {
        const float f = ml[c][0] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml[c][0] - mp) * ml[c][1];
        l += f;
#pragma unroll
        for (int gh = 0; gh < 2; ++gh)
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            const uint32_t d0 = v[c][gh][2 * q], d1 = v[c][gh][2 * q + 1];
            acc[2 * gh + q] += f * f4{half_lo(d0), half_hi(d0), half_lo(d1), half_hi(d1)};
          }
      }
    }
    m = mp;
  }
  // Output: the block of dims 32db..32db+31 of this wave's rows (lanes l and l^32: row l % 32).
  const float inv = l > 0.f ? 1.f / l : 0.f;  // l: the chunks' whole-row sums
  const int S = w.seq_len, head = (w.seq_kvh & 15) * kGroup + (wave >> 1);
  const int q_pos = w.q_block * kBlockQ + (wave & 1) * kWaveQ + lq;
  const uint32_t ostride_b = p.o_stride_b;
  const auto ors = make_rsrc(reinterpret_cast<const char*>(p.o) + (uint64_t)w.seq_start * ostride_b + head * kRowBytes,
                             (uint32_t)S * ostride_b);
  const auto lrs = make_rsrc(p.o_last + (int64_t)(w.seq_kvh >> 4) * (kQHeads * kHeadDim) + head * kHeadDim,
                             p.o_last ? kRowBytes : 0u);
  const uint32_t orow = (q_pos < S ? (uint32_t)q_pos * ostride_b : 0x80000000u) + 16u * hl;
  const uint32_t lrow = (q_pos == S - 1 ? 0u : 0x80000000u) + 16u * hl;
  typedef uint32_t u4 __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int gp = 0; gp < 2; ++gp) {
    const f4 va = acc[2 * gp], vb = acc[2 * gp + 1];
    const uint32_t a0 = pack2(va[0] * inv, va[1] * inv), a1 = pack2(va[2] * inv, va[3] * inv);
    const uint32_t b0 = pack2(vb[0] * inv, vb[1] * inv), b1 = pack2(vb[2] * inv, vb[3] * inv);
    const auto r0 = __builtin_amdgcn_permlane32_swap(a0, b0, false, false);
    const auto r1 = __builtin_amdgcn_permlane32_swap(a1, b1, false, false);
    const u4 val = {r0[0], r1[0], r0[1], r1[1]};
    const uint32_t d = 2u * (32 * db + 16 * gp);
    __builtin_amdgcn_raw_buffer_store_b128(val, lrs, lrow + d, 0, 0);
    __builtin_amdgcn_raw_buffer_store_b128(val, ors, orow + d, 0, 0);
  }
}

hipError_t launch_attn_merge(const AttnParams& p, hipStream_t stream) {
  if (p.n_splits <= 0) return hipSuccess;
  hipLaunchKernelGGL(attn_merge_kernel, dim3(p.n_splits * kWaves), dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

// Retained-key bitmask of one sequence through the kernel's own key iteration (kept_keys_row):
// one thread per query row.
__global__ void debug_mask_kernel(int S, MaskSpec mask, uint32_t* bits, int words_per_row) {
  const int q = blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= S) return;
  kept_keys_row(q, S, mask, bits + (int64_t)q * words_per_row, words_per_row);
}

hipError_t launch_attn_fwd(const AttnParams& p, hipStream_t stream) {
  if (p.n_slots <= 0) return hipSuccess;
  // Plans without split items run the variant without the partial-result path (fewer live
  // registers in the tile loop).
  const dim3 grid(p.n_slots), block(kThreads);
  if (p.timeline) {
    if (p.n_splits > 0) hipLaunchKernelGGL((attn_fwd_kernel<true, false, false, true>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((attn_fwd_kernel<false, false, false, true>), grid, block, 0, stream, p);
    return hipGetLastError();
  }
  if (p.maskbits) {
    if (p.n_splits > 0) hipLaunchKernelGGL((attn_fwd_kernel<true, false, true>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((attn_fwd_kernel<false, false, true>), grid, block, 0, stream, p);
    return hipGetLastError();
  }
  if (p.n_splits > 0) {
    if (p.o_last) hipLaunchKernelGGL((attn_fwd_kernel<true, true>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((attn_fwd_kernel<true, false>), grid, block, 0, stream, p);
  } else {
    if (p.o_last) hipLaunchKernelGGL((attn_fwd_kernel<false, true>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((attn_fwd_kernel<false, false>), grid, block, 0, stream, p);
  }
  return hipGetLastError();
}

// XCD (XCC) of each workgroup of a launch shaped like the attention kernel's (256 threads,
// 64 KiB LDS): out[b] = hardware XCC_ID of workgroup b.
__global__ __launch_bounds__(kThreads, 2) void xcd_map_kernel(int* out) {
  __shared__ char lds[kTileBytes * 4];
  unsigned x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  lds[threadIdx.x] = 0;
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = (int)(x & 0xf) + lds[1];
}

hipError_t launch_xcd_map(int* out, int n, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(xcd_map_kernel, dim3(n), dim3(kThreads), 0, stream, out);
  return hipGetLastError();
}

hipError_t launch_debug_mask(int S, MaskSpec mask, uint32_t* bits, int words_per_row,
                             hipStream_t stream) {
  if (S <= 0) return hipSuccess;
  hipLaunchKernelGGL(debug_mask_kernel, dim3((S + 255) / 256), dim3(256), 0, stream, S, mask,
                     bits, words_per_row);
  return hipGetLastError();
}

}  // namespace qattn
