// attn_fwd.hip -- causal / prefix+local GQA prefill attention for gfx950 (MI355X).
//
// Replaces the reference's tiled flash attention shader (src/webgpu/ops.ts:168-241).  Same
// result (softmax(mask(QK^T)/sqrt(128)) V per query head, mask ops.ts:205-209,220), computed
// the CDNA4 way:
//   * one workgroup = (sequence, KV head, 64 query positions) and BOTH query heads of the GQA
//     group (4 wavefronts x 32 rows), so each K/V tile is staged in LDS once for two heads;
//   * S^T = K Q^T and O^T = V^T P^T on v_mfma_f32_32x32x16_f16 (fp16 in, fp32 accumulate), so
//     every lane owns one query row: the online-softmax row max / sum need one cross-lane swap
//     (lane l <-> l^32) instead of a 16-thread serial loop;
//   * Q stays in registers for the whole key loop; K/V tiles are double buffered in LDS with
//     the next tile's global loads in flight during the current tile's MFMAs;
//   * causal and prefix/local masks skip whole key tiles (key_tiles), and element masks run only
//     on tiles that straddle a boundary (tile_full);
//   * packed varlen sequences (cu_seqlens): no padded rows, no padded keys.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_common.h"

namespace qattn {

typedef _Float16 half_t;
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16x __attribute__((ext_vector_type(16)));

constexpr int kKStride = kHeadDim + 8;  // K tile row stride in halves (272 B): 4-bank skew/row
constexpr int kVStride = kTileK + 4;    // V^T tile row stride in halves (136 B)

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

__global__ __launch_bounds__(kThreads, 2) void attn_fwd_kernel(AttnParams p) {
  __shared__ __attribute__((aligned(16))) half_t sK[2][kTileK * kKStride];
  __shared__ __attribute__((aligned(16))) half_t sV[2][kHeadDim * kVStride];

  const WorkItem w = p.work[blockIdx.x];
  const int seq_start = w.seq_start;
  const int S = w.seq_len;
  const int kvh = w.seq_kvh & 15;
  const int seq = w.seq_kvh >> 4;
  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int lq = lane & 31;  // query row of this lane inside the wave's 32-row tile
  const int hl = lane >> 5;  // which half of the MFMA K dimension this lane feeds
  const int head = kvh * kGroup + (wave >> 1);
  const int blk_q0 = w.q_block * kBlockQ;
  const int blk_q1 = min(S, blk_q0 + kBlockQ) - 1;
  const int wq0 = blk_q0 + (wave & 1) * kWaveQ;   // first query position of this wave
  const int wq1 = min(S - 1, wq0 + kWaveQ - 1);   // last valid one (wq1 < wq0: idle wave)
  const bool wave_live = wq0 < S;
  const int q_pos = wq0 + lq;
  const MaskSpec mask = p.mask;

  // ---- Q fragment in registers: B operand of S^T = K Q^T (lane: row q, 8 consecutive d) ----
  h8 qreg[8];
  {
    const half_t* qrow = p.q + (int64_t)(seq_start + q_pos) * p.q_stride + head * kHeadDim + 8 * hl;
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      h8 z = {};
      qreg[st] = (q_pos < S) ? *reinterpret_cast<const h8*>(qrow + 16 * st) : z;
    }
  }

  const half_t* kbase = p.k + (int64_t)seq_start * p.k_stride + kvh * kHeadDim;
  const half_t* vbase = p.v + (int64_t)seq_start * p.v_stride + kvh * kHeadDim;

  // Register staging of the next K/V tile.  K: 4 x 16 B per thread, row-major copy.
  // V: 4 keys x 8 dims per thread, transposed into V^T on the LDS store.
  h8 kreg[4], vreg[4];
  const int v_kg = tid >> 4;        // key group: keys 4*v_kg .. 4*v_kg+3
  const int v_d = (tid & 15) * 8;   // dims v_d .. v_d+7
  auto gload = [&](int kt) {
    const int kb = kt * kTileK;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = tid + kThreads * j;
      const int key = kb + (c >> 4);
      h8 z = {};
      kreg[j] = key < S ? *reinterpret_cast<const h8*>(kbase + (int64_t)key * p.k_stride + (c & 15) * 8) : z;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = kb + 4 * v_kg + i;
      h8 z = {};
      vreg[i] = key < S ? *reinterpret_cast<const h8*>(vbase + (int64_t)key * p.v_stride + v_d) : z;
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int c = tid + kThreads * j;
      *reinterpret_cast<h8*>(&sK[buf][(c >> 4) * kKStride + (c & 15) * 8]) = kreg[j];
    }
#pragma unroll
    for (int di = 0; di < 8; ++di) {
      h4 t = {vreg[0][di], vreg[1][di], vreg[2][di], vreg[3][di]};
      *reinterpret_cast<h4*>(&sV[buf][(v_d + di) * kVStride + 4 * v_kg]) = t;
    }
  };

  // Online-softmax state of this lane's row (base-2 domain) and the O^T accumulator.
  float m_run = -INFINITY;
  float l_run = 0.f;
  f16x o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db] = f16x{};

  const TileRanges tiles = key_tiles(blk_q0, blk_q1, S, mask);
  const int ntiles = tiles.count();

  gload(tiles.at(0));
  sstore(0);
  __syncthreads();

  for (int it = 0; it < ntiles; ++it) {
    const int buf = it & 1;
    const int kb = tiles.at(it) * kTileK;
    if (it + 1 < ntiles) gload(tiles.at(it + 1));

    if (wave_live && tile_any(kb, wq0, wq1, S, mask)) {
      // ---- S^T (64 keys x 32 queries) = K (64 x 128) . Q^T ----
      f16x s0 = {}, s1 = {};
      const half_t* ka = &sK[buf][lq * kKStride + 8 * hl];
      const half_t* kc = &sK[buf][(32 + lq) * kKStride + 8 * hl];
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        s0 = mfma32(*reinterpret_cast<const h8*>(ka + 16 * st), qreg[st], s0);
        s1 = mfma32(*reinterpret_cast<const h8*>(kc + 16 * st), qreg[st], s1);
      }
      // Lane holds S^T[key][q_pos] for key = kb + 32*(r>>4) + 8*((r&15)>>2) + 4*hl + (r&3).
      float sv[32];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        sv[r] = s0[r];
        sv[16 + r] = s1[r];
      }
      if (!tile_full(kb, wq0, wq1, S, mask)) {
#pragma unroll
        for (int r = 0; r < 32; ++r) {
          const int key = kb + 32 * (r >> 4) + 8 * ((r & 15) >> 2) + 4 * hl + (r & 3);
          if (!retained(q_pos, key, S, mask)) sv[r] = -INFINITY;
        }
      }
      float mx = sv[0];
#pragma unroll
      for (int r = 1; r < 32; ++r) mx = fmaxf(mx, sv[r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(m_run, mx * p.scale_log2);
      const float m_use = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
      float psum = 0.f;
#pragma unroll
      for (int r = 0; r < 32; ++r) {
        sv[r] = __builtin_amdgcn_exp2f(fmaf(sv[r], p.scale_log2, -m_use));
        psum += sv[r];
      }
      l_run = l_run * alpha + psum;
      m_run = m_new;
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db] *= alpha;

      // ---- O^T (128 d x 32 q) += V^T (128 x 64 keys) . P^T ----
      // MFMA step t covers keys kb+16t..kb+16t+15; slot j of lane half hl is key
      // 16t + 8*(j>>2) + 4*hl + (j&3), which is exactly where P sits in sv[8t + j].
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        h8 pf;
#pragma unroll
        for (int j = 0; j < 8; ++j) pf[j] = (half_t)sv[8 * t + j];
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const half_t* vp = &sV[buf][(32 * db + lq) * kVStride + 16 * t + 4 * hl];
          const h4 lo = *reinterpret_cast<const h4*>(vp);
          const h4 hi = *reinterpret_cast<const h4*>(vp + 8);
          const h8 va = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          o[db] = mfma32(va, pf, o[db]);
        }
      }
    }

    if (it + 1 < ntiles) sstore(buf ^ 1);
    __syncthreads();
  }

  // ---- epilogue: O = O^T / l, lane owns row q_pos, dims 32db + 8g + 4hl + 0..3 ----
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (wave_live && q_pos < S) {
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
