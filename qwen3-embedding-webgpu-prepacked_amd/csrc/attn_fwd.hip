// attn_fwd.hip -- causal / prefix+local GQA prefill attention for gfx950 (MI355X).
//
// Replaces the reference's tiled flash attention shader (src/webgpu/ops.ts:168-241).  Same
// result (softmax(mask(QK^T)/sqrt(128)) V per query head, mask ops.ts:205-209,220), computed
// the CDNA4 way:
//   * one workgroup = (sequence, KV head, 64 query positions) and BOTH query heads of the GQA
//     group (4 wavefronts x 32 rows), so each K/V tile is staged in LDS once for two heads;
//   * S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_32x32x16_f16 (fp16 in, fp32 accumulate), so
//     every lane owns one query row: the row max / row sum need one permlane32 swap;
//   * K/V tiles go HBM -> LDS with buffer_load ... lds (no staging registers); the buffer
//     resource spans only the sequence's rows, so keys past its end arrive as zeros;
//   * LDS tiles are row-major 256 B rows with a 16 B-granular XOR swizzle chosen so that the K
//     fragment reads (ds_read_b128) and the V^T fragment reads (ds_read_b64_tr_b16, the gfx950
//     LDS transpose load) are bank-conflict free;
//   * software pipelined: iteration j issues the S^T MFMAs of tile j+1 and the PV MFMAs of tile
//     j-1 in the same basic block as the softmax VALU work of tile j, so the matrix cores and
//     the VALU run side by side; the score / probability registers alternate between two sets
//     by iteration parity (no copies); K and V are double buffered in LDS;
//   * lazy rescaling: O and l are rescaled only when a row max grows by more than 2^8;
//   * causal and prefix/local masks skip whole key tiles (key_tiles); element masks run only on
//     tiles that straddle a boundary (tile_full).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "attn_common.h"

namespace qattn {

typedef _Float16 half_t;
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
constexpr float kRescaleThreshold = 8.0f;                    // log2 units

struct AttnParams {
  const half_t* q;
  const half_t* k;
  const half_t* v;  // already offset by v_offset
  half_t* o;
  half_t* o_last;
  int64_t q_stride, k_stride, v_stride, o_stride;
  const WorkItem* work;
  int32_t n_work;
  MaskSpec mask;
  float scale_log2;  // (1/sqrt(128)) * log2(e)
};

__device__ inline f16x mfma32(h8 a, h8 b, f16x c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Raw buffer resource over `bytes` bytes at `base`; loads past the end return zeros.
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

__global__ __launch_bounds__(kThreads, 2) void attn_fwd_kernel(AttnParams p) {
  // K and V tiles, double buffered, 16 KiB each.  Four distinct objects (not offsets into one
  // array) with buffer choices fixed at compile time, so the compiler can see that the LDS-DMA
  // loads in flight never alias the tile being read and does not wait for them.
  __shared__ __attribute__((aligned(1024))) char sK0[kTileBytes];
  __shared__ __attribute__((aligned(1024))) char sK1[kTileBytes];
  __shared__ __attribute__((aligned(1024))) char sV0[kTileBytes];
  __shared__ __attribute__((aligned(1024))) char sV1[kTileBytes];

  const WorkItem w = p.work[blockIdx.x];
  const int seq_start = w.seq_start;
  const int S = w.seq_len;
  const int kvh = w.seq_kvh & 15;
  const int seq = w.seq_kvh >> 4;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: keeps rsrc/M0 in SGPRs
  const int lane = tid & 63;
  const int lq = lane & 31;  // query row of this lane inside the wave's 32-row tile
  const int hl = lane >> 5;  // which half of the MFMA K dimension this lane feeds
  const int head = kvh * kGroup + (wave >> 1);
  const int blk_q0 = w.q_block * kBlockQ;
  const int blk_q1 = min(S, blk_q0 + kBlockQ) - 1;
  const int wq0 = blk_q0 + (wave & 1) * kWaveQ;
  const int wq1 = min(S - 1, wq0 + kWaveQ - 1);
  const int q_pos = wq0 + lq;
  const MaskSpec mask = p.mask;
  const int ps = min(S, mask.prefix);
  const int ws = min(S, mask.window);
  const float c = p.scale_log2;

  // ---- Q fragment (B operand of S^T = K Q^T): lane = query row, 8 consecutive dims per step.
  h8 qreg[8];
  {
    const half_t* qhead = p.q + (int64_t)seq_start * p.q_stride + head * kHeadDim;
    const auto rs = make_rsrc(qhead, (uint32_t)S * (uint32_t)p.q_stride * 2u);
    const uint32_t row_off = (uint32_t)q_pos * (uint32_t)p.q_stride * 2u + 16u * hl;
#pragma unroll
    for (int st = 0; st < 8; ++st)
      qreg[st] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(rs, row_off + 32u * st, 0, 0));
  }

  // ---- tile loads: kLoadsPerTile buffer_load...lds per lane per tile; instruction j of wave
  // `wave` fills LDS rows 16j + 4*wave .. +3 (1 KiB, lane-contiguous).  Lane writes physical chunk
  // lane&15 of row r with the logical 16 B chunk (lane&15) ^ swizzle(r) of key row kb + r.
  const char* kbase = reinterpret_cast<const char*>(p.k + (int64_t)seq_start * p.k_stride + kvh * kHeadDim);
  const char* vbase = reinterpret_cast<const char*>(p.v + (int64_t)seq_start * p.v_stride + kvh * kHeadDim);
  const uint32_t kstride_b = (uint32_t)p.k_stride * 2u, vstride_b = (uint32_t)p.v_stride * 2u;
  uint32_t koff[kLoadsPerTile], voff[kLoadsPerTile];
#pragma unroll
  for (int j = 0; j < kLoadsPerTile; ++j) {
    const int r = 16 * j + 4 * wave + (lane >> 4);
    const int pc = lane & 15;
    koff[j] = (uint32_t)r * kstride_b + (uint32_t)((pc ^ (r & 15)) << 4);
    voff[j] = (uint32_t)r * vstride_b + (uint32_t)((pc ^ ((r & 3) << 1)) << 4);
  }
  auto load_tile = [&](char* dst, const char* base, uint32_t stride_b, const uint32_t* off, int kt) {
    const int kb = kt * kTileK;
    const auto rs = make_rsrc(base + (int64_t)kb * stride_b, (uint32_t)(S - kb) * stride_b);
#pragma unroll
    for (int j = 0; j < kLoadsPerTile; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(dst + j * 4096 + wave * 1024), 16,
                                               off[j], 0, 0, 0);
  };

  // ---- LDS read addresses.
  // K (A operand of S^T): lane reads key row lq (+32 for the second block), logical chunk
  // 2*st + hl, stored at physical chunk (2*st + hl) ^ (lq & 15).
  uint32_t kread[8];
#pragma unroll
  for (int st = 0; st < 8; ++st) kread[st] = lq * kRowBytes + (((2 * st + hl) ^ (lq & 15)) << 4);
  // V^T (A operand of O^T = V^T P^T) through ds_read_b64_tr_b16: in each 16-lane group G the
  // source lane a reads 4 halves at key row 4*(G>>1) + (a>>2) (+16t, +8 for slots 4..7), dims
  // 32db + 16(G&1) + 4(a&3); lane a then receives V[4 keys][dim 32db + 16(G&1) + a].
  uint32_t vread[4];
  {
    const int a = lane & 15, G = lane >> 4;
    const int row = 4 * (G >> 1) + (a >> 2);
#pragma unroll
    for (int db = 0; db < 4; ++db) {
      const int chunk = (4 * db + 2 * (G & 1) + ((a & 3) >> 1)) ^ ((a >> 2) << 1);
      vread[db] = row * kRowBytes + (chunk << 4) + ((a & 1) << 3);
    }
  }

  // S^T (64 keys x 32 queries) for the K tile in `kt`.  Lane holds S^T[key][q_pos] for
  // key = kb + 4*hl + key_off(r), r = 0..31 over (s[0], s[1]).
  auto qk = [&](const char* kt, f16x (&s)[2]) {
    s[0] = f16x{};
    s[1] = f16x{};
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const h8 a0 = *reinterpret_cast<const h8*>(kt + kread[st]);
      const h8 a1 = *reinterpret_cast<const h8*>(kt + kread[st] + 32 * kRowBytes);
      s[0] = mfma32(a0, qreg[st], s[0]);
      s[1] = mfma32(a1, qreg[st], s[1]);
    }
  };

  // O^T (128 d x 32 q) += V^T (128 x 64 keys) . P^T.  Step t covers keys kb+16t..kb+16t+15;
  // slot j of lane half hl is key 16t + 8*(j>>2) + 4*hl + (j&3), whose probability is pf[t][j].
  f16x o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db] = f16x{};
  auto pv = [&](const char* vt, const h8 (&pf)[4]) {
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4_t*)(vt + vread[db] + t * 4096));
        const s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4_t*)(vt + vread[db] + t * 4096 + 2048));
        const h4 lo_h = __builtin_bit_cast(h4, lo), hi_h = __builtin_bit_cast(h4, hi);
        const h8 va = {lo_h[0], lo_h[1], lo_h[2], lo_h[3], hi_h[0], hi_h[1], hi_h[2], hi_h[3]};
        o[db] = mfma32(va, pf[t], o[db]);
      }
    }
  };

  // Element mask of a boundary tile (keys that keep_key() drops become -inf).
  auto apply_mask = [&](f16x (&s)[2], int kb) {
    const int kl = kb + 4 * hl;
#pragma unroll
    for (int r = 0; r < 32; ++r)
      if (!keep_key(q_pos, kl + key_off(r), ps, ws, mask.kind)) s[r >> 4][r & 15] = -INFINITY;
  };

  // Online softmax of this lane's row over one tile's 64 scores -> fp16 P; returns whether the
  // row max moved by more than the lazy-rescale threshold (then O must be scaled by alpha).
  float m_run = -INFINITY;  // max (log2 domain) the probabilities are taken against
  float l_run = 0.f;        // running sum of the fp16-rounded probabilities
  auto softmax = [&](const f16x (&s)[2], h8 (&pf)[4], float& alpha) {
    float mx = fmaxf(fmaxf(s[0][0], s[0][1]), s[0][2]);
#pragma unroll
    for (int r = 3; r < 31; r += 2) mx = fmaxf(fmaxf(mx, s[r >> 4][r & 15]), s[(r + 1) >> 4][(r + 1) & 15]);
    mx = fmaxf(mx, s[1][15]);
    mx = pair_max(mx);
    const float m_cand = fmaxf(m_run, mx * c);
    const bool need = m_cand > m_run + kRescaleThreshold;
    const float m_next = need ? m_cand : m_run;
    const float m_use = m_next == -INFINITY ? 0.f : m_next;
    alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    // P in fp16 feeds the PV MFMA; the row sum adds those same rounded values (exactly, via
    // v_dot2 against 1.0), so O is an exact weighted mean of V and the fp16 rounding of P only
    // perturbs the weights.
    float psum = 0.f;
    const h2 ones = {(half_t)1.0f, (half_t)1.0f};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int r = 8 * t + j;
        pf[t][j] = (half_t)__builtin_amdgcn_exp2f(fmaf(s[r >> 4][r & 15], c, -m_use));
      }
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        const h2 pair = {pf[t][j], pf[t][j + 1]};
        psum = __builtin_amdgcn_fdot2(pair, ones, psum, false);
      }
    }
    m_run = m_next;
    l_run = l_run * alpha + psum;
    return need;
  };
  auto rescale = [&](bool need, float alpha) {
    if (__builtin_amdgcn_ballot_w64(need) != 0) {
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db] *= alpha;
    }
  };

  const TileRanges tiles = key_tiles(blk_q0, blk_q1, S, mask);
  const int ntiles = tiles.count();

  // Two register sets for scores / probabilities, alternating by iteration parity.
  f16x sA[2], sB[2];
  h8 pA[4], pB[4];

  // Prologue: K(0), K(1) resident; S(0) computed.
  load_tile(sK0, kbase, kstride_b, koff, tiles.at(0));
  if (ntiles > 1) load_tile(sK1, kbase, kstride_b, koff, tiles.at(1));
  __builtin_amdgcn_s_waitcnt(0);  // (gfx9 encoding 0: vmcnt/expcnt/lgkmcnt all zero)
  __syncthreads();
  qk(sK0, sA);

  // Iteration `it`, B = it & 1 (compile time).  Before it: S(it) in s_cur, P(it-1) in p_prev,
  // K(it+1) in sK<B^1>, V(it-1) in sV<B^1>.  It refills sK<B> with K(it+2) and sV<B> with V(it),
  // computes S(it+1) into s_nxt (stale-buffer garbage on the last tile, never used), adds
  // P(it-1) V(it-1) to O and turns S(it) into P(it) in p_cur.
  auto body = [&](auto bconst, int it, f16x (&s_cur)[2], f16x (&s_nxt)[2], h8 (&p_cur)[4],
                  const h8 (&p_prev)[4], bool with_pv) {
    constexpr int B = decltype(bconst)::value;
    char* const kfree = B == 0 ? sK0 : sK1;
    char* const knext = B == 0 ? sK1 : sK0;
    char* const vfree = B == 0 ? sV0 : sV1;
    char* const vprev = B == 0 ? sV1 : sV0;
    const int kb = tiles.at(it) * kTileK;
    // Loads issued last iteration have landed and every wavefront is done with last
    // iteration's reads of the buffers about to be refilled.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (it + 2 < ntiles) load_tile(kfree, kbase, kstride_b, koff, tiles.at(it + 2));
    load_tile(vfree, vbase, vstride_b, voff, tiles.at(it));
    if (!tile_full(kb, wq0, wq1, S, mask)) apply_mask(s_cur, kb);
    qk(knext, s_nxt);
    if (with_pv) pv(vprev, p_prev);
    float alpha;
    const bool need = softmax(s_cur, p_cur, alpha);
    // Keep P(it) and the row sum computed here, beside the MFMAs above: without this use the
    // compiler sinks the exponentials below the rescale branch, where no MFMA work overlaps them.
    asm volatile("" ::"v"(p_cur[0]), "v"(p_cur[1]), "v"(p_cur[2]), "v"(p_cur[3]), "v"(l_run));
    rescale(need, alpha);
  };

  body(std::integral_constant<int, 0>{}, 0, sA, sB, pA, pB, false);
  for (int it = 1; it < ntiles; it += 2) {
    body(std::integral_constant<int, 1>{}, it, sB, sA, pB, pA, true);
    if (it + 1 < ntiles) body(std::integral_constant<int, 0>{}, it + 1, sA, sB, pA, pB, true);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if ((ntiles - 1) & 1)
    pv(sV1, pB);
  else
    pv(sV0, pA);

  // ---- epilogue: O = O^T / l, lane owns row q_pos, dims 32db + 8g + 4hl + 0..3 ----
  const float l_tot = pair_sum(l_run);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (q_pos < S) {
    half_t* orow = p.o + (int64_t)(seq_start + q_pos) * p.o_stride + head * kHeadDim;
    half_t* lrow = (p.o_last && q_pos == S - 1) ? p.o_last + (int64_t)seq * (kQHeads * kHeadDim) + head * kHeadDim : nullptr;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const h4 val = {(half_t)(o[db][4 * g + 0] * inv), (half_t)(o[db][4 * g + 1] * inv),
                        (half_t)(o[db][4 * g + 2] * inv), (half_t)(o[db][4 * g + 3] * inv)};
        const int d = 32 * db + 8 * g + 4 * hl;
        *reinterpret_cast<h4*>(orow + d) = val;
        if (lrow) *reinterpret_cast<h4*>(lrow + d) = val;
      }
  }
}

// Retained-key bitmask of one sequence through the kernel's own key iteration (kept_keys_row):
// one thread per query row.
__global__ void debug_mask_kernel(int S, MaskSpec mask, uint32_t* bits, int words_per_row) {
  const int q = blockIdx.x * blockDim.x + threadIdx.x;
  if (q >= S) return;
  kept_keys_row(q, S, mask, bits + (int64_t)q * words_per_row, words_per_row);
}

hipError_t launch_attn_fwd(const AttnParams& p, hipStream_t stream) {
  if (p.n_work <= 0) return hipSuccess;
  hipLaunchKernelGGL(attn_fwd_kernel, dim3(p.n_work), dim3(kThreads), 0, stream, p);
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
