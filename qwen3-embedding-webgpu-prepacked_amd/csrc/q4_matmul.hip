// q4_matmul.hip -- Q4_0 "tile32-compact" dequant-GEMM: Y = X W^T with fp16 activations X [M, K]
// and 4-bit weights W [N, K], the projection that produces the attention path's Q/K/V rows.
//
// Replaces the reference's compact batch matmul (src/webgpu/quant-matmul.ts:267-307, dequant
// :99-108) over the layout written by packQ40Tile32 (src/prepacked/format.ts:64-96): 20-byte
// records (f16 scale, 2 pad bytes, 16 quant bytes; element j of the 32-column block in the low
// nibble of byte j, element j+16 in its high nibble) ordered ((n/32) * (K/32) + k/32) * 32 + n%32.
// The weight is f16(scale * (q - 8)), as the reference dequantises it; the products and sums run
// in fp32 on the matrix cores (the reference accumulates in f16).
//
// The CDNA4 shape:
//   * workgroup tile 128 (M) x 128 (N), four wavefronts of 64 x 64, each 2 x 2 blocks of
//     v_mfma_f32_32x32x16_f16 with fp32 accumulators (64 VGPRs);
//   * per 32-column K block a lane loads its A fragments straight from X (four 16-byte loads:
//     rows of 32 consecutive halves are contiguous) and, for each of its two N blocks, one
//     weight record's scale word and the 8 quant bytes its B fragment needs; the nibbles become
//     f16 by bit-OR into 1024.0 (f16(1024 + q)), an exact subtract of 1032 and one f16 multiply
//     by the scale (the same single rounding as the reference's f16 product);
//   * a 4-stage register pipeline: the loads of K block kb + 3 are issued before block kb's 8
//     MFMAs, into the stage that block kb - 1 just freed (stages are compile-time register sets,
//     so nothing is copied, and every load is issued -- past the last block it re-reads the last
//     block -- so the compiler's wait counts are the same on every path);
//   * tiles are numbered so that consecutive workgroups on one XCD (workgroup b runs on XCD
//     b % 8) walk the N tiles of one M tile: its X rows stay in that XCD's L2.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace qattn {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int kQ4Tile = 128;    // workgroup tile, both dimensions
constexpr int kQ4Record = 20;   // bytes per (row, 32-column block)

__device__ inline __amdgpu_buffer_rsrc_t q4_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// Two f16 weights from the low (HIGH = false) or high nibbles of bytes 0 and 1 of `pair`
// (laid out as byte 0 in bits 0..7 and byte 1 in bits 16..23): f16(scale * (q - 8)).
template <bool HIGH>
__device__ inline h2 dequant2(uint32_t pair, h2 scale) {
  const uint32_t q = (HIGH ? pair >> 4 : pair) & 0x000F000Fu;
  const h2 biased = __builtin_bit_cast(h2, q | 0x64006400u);  // 1024 + q, exact
  const h2 centred = biased - h2{(_Float16)1032.0f, (_Float16)1032.0f};  // q - 8, exact
  return centred * scale;  // one rounding, as the reference's f16 multiply
}

// The 8 weights of a B fragment: quant bytes b0..b7 (two dwords) -> low or high nibbles.
template <bool HIGH>
__device__ inline h8 dequant8(u2 q, h2 scale) {
  // byte pairs (b0,b1), (b2,b3) of each dword into the two 16-bit halves
  const uint32_t p0 = __builtin_amdgcn_perm(0u, q[0], 0x0C010C00u);
  const uint32_t p1 = __builtin_amdgcn_perm(0u, q[0], 0x0C030C02u);
  const uint32_t p2 = __builtin_amdgcn_perm(0u, q[1], 0x0C010C00u);
  const uint32_t p3 = __builtin_amdgcn_perm(0u, q[1], 0x0C030C02u);
  const h2 a = dequant2<HIGH>(p0, scale), b = dequant2<HIGH>(p1, scale);
  const h2 c = dequant2<HIGH>(p2, scale), d = dequant2<HIGH>(p3, scale);
  return h8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

__global__ __launch_bounds__(256, 2) void q4_matmul_kernel(const _Float16* __restrict__ x, int64_t ldx, int M, int K,
                                                           const uint8_t* __restrict__ w, uint32_t w_bytes, int N,
                                                           _Float16* __restrict__ y, int64_t ldy, int tiles_n,
                                                           int tiles_total, int per_xcd) {
  // Tile of this workgroup: XCD b % 8 owns tiles [xcd * per_xcd, (xcd + 1) * per_xcd).
  const int b = blockIdx.x;
  const int t = (b & 7) * per_xcd + (b >> 3);
  if (b >> 3 >= per_xcd || t >= tiles_total) return;
  const int m0 = (t / tiles_n) * kQ4Tile, n0 = (t % tiles_n) * kQ4Tile;

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int l32 = lane & 31, hl = lane >> 5;
  const int wm = m0 + 64 * (wave & 1), wn = n0 + 64 * (wave >> 1);
  const int kblocks = K >> 5;

  // X rows of the run (rows >= M read as zeros), the weight tensor, Y rows.
  const auto xrs = q4_rsrc(x, (uint32_t)M * (uint32_t)ldx * 2u);
  const auto wrs = q4_rsrc(w, w_bytes);
  const auto yrs = q4_rsrc(y, (uint32_t)M * (uint32_t)ldy * 2u);

  // A fragment (mb, s): row wm + 32 mb + l32, columns 32 kb + 16 s + 8 hl .. +7.
  uint32_t a_off[2];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) a_off[mb] = (uint32_t)(wm + 32 * mb + l32) * (uint32_t)ldx * 2u + 16u * hl;
  // Weight record of (row n = wn + 32 nb + l32, block kb): (((n / 32) * kblocks + kb) * 32 + l32) * 20.
  uint32_t w_off[2];
#pragma unroll
  for (int nb = 0; nb < 2; ++nb)
    w_off[nb] = ((uint32_t)((wn >> 5) + nb) * (uint32_t)kblocks * 32u + (uint32_t)l32) * kQ4Record;
  const uint32_t w_step = 32u * kQ4Record;  // next K block of the same row

  auto load = [&](int kb, h8 (&a)[2][2], uint32_t (&sc)[2], u2 (&q)[2]) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int s = 0; s < 2; ++s)
        a[mb][s] = __builtin_bit_cast(
            h8, __builtin_amdgcn_raw_buffer_load_b128(xrs, a_off[mb] + (uint32_t)kb * 64u + 32u * s, 0, 0));
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const uint32_t r = w_off[nb] + (uint32_t)kb * w_step;
      sc[nb] = __builtin_amdgcn_raw_buffer_load_b32(wrs, r, 0, 0);
      q[nb] = __builtin_amdgcn_raw_buffer_load_b64(wrs, r + 4u + 8u * hl, 0, 0);
    }
  };

  f16x acc[2][2];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = f16x{};

  constexpr int kStages = 4;
  h8 a[kStages][2][2];
  uint32_t sc[kStages][2];
  u2 q[kStages][2];
  auto load_stage = [&](auto sconst, int kb) {
    constexpr int S = decltype(sconst)::value;
    load(kb < kblocks ? kb : kblocks - 1, a[S], sc[S], q[S]);
  };
  auto compute_stage = [&](auto sconst) {
    constexpr int S = decltype(sconst)::value;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const _Float16 s = __builtin_bit_cast(h2, sc[S][nb])[0];
      const h2 scale = {s, s};
      const h8 b_lo = dequant8<false>(q[S][nb], scale);  // columns 8 hl .. +7 of the block
      const h8 b_hi = dequant8<true>(q[S][nb], scale);   // columns 16 + 8 hl .. +7
#pragma unroll
      for (int mb = 0; mb < 2; ++mb) {
        acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[S][mb][0], b_lo, acc[mb][nb], 0, 0, 0);
        acc[mb][nb] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[S][mb][1], b_hi, acc[mb][nb], 0, 0, 0);
      }
    }
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  using S3 = std::integral_constant<int, 3>;
  // Step kb: issue block kb + 3 into stage (kb + 3) % 4, then compute block kb from stage kb % 4.
  auto step = [&](auto cur, auto ahead, int kb) {
    load_stage(ahead, kb + 3);
    if (kb < kblocks) compute_stage(cur);
  };
  // Prologue in stage order (the scheduler may not interleave the stages: the loop's waits count
  // on stage 0 being the oldest in flight on entry, as it is on every back edge).
  load_stage(S0{}, 0);
  __builtin_amdgcn_sched_barrier(0);
  load_stage(S1{}, 1);
  __builtin_amdgcn_sched_barrier(0);
  load_stage(S2{}, 2);
  __builtin_amdgcn_sched_barrier(0);
  for (int kb = 0; kb < kblocks; kb += kStages) {
    step(S0{}, S3{}, kb);
    step(S1{}, S0{}, kb + 1);
    step(S2{}, S1{}, kb + 2);
    step(S3{}, S2{}, kb + 3);
  }

  // D (32 x 32 per block): lane holds column l32 and rows 8 (r / 4) + 4 hl + r % 4, r = 0..15.
  // Columns >= N are skipped here; rows >= M fall outside the Y resource and are dropped.
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int n = wn + 32 * nb + l32;
    if (n < N) {
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = wm + 32 * mb + 8 * (r >> 2) + 4 * hl + (r & 3);
          const uint32_t off = m < M ? ((uint32_t)m * (uint32_t)ldy + (uint32_t)n) * 2u : 0x80000000u;
          __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, (_Float16)acc[mb][nb][r]), yrs,
                                                off, 0, 0);
        }
    }
  }
}

// Grid: 8 * ceil(tiles / 8) workgroups of 256 threads (the surplus ones exit at once).
hipError_t launch_q4_matmul(const _Float16* x, int64_t ldx, int M, int K, const uint8_t* w, uint32_t w_bytes, int N,
                            _Float16* y, int64_t ldy, hipStream_t stream) {
  if (M <= 0 || N <= 0) return hipSuccess;
  const int tiles_m = (M + kQ4Tile - 1) / kQ4Tile, tiles_n = (N + kQ4Tile - 1) / kQ4Tile;
  const int tiles = tiles_m * tiles_n, per_xcd = (tiles + 7) / 8;
  hipLaunchKernelGGL(q4_matmul_kernel, dim3((unsigned)(8 * per_xcd)), dim3(256), 0, stream, x, ldx, M, K, w, w_bytes,
                     N, y, ldy, tiles_n, tiles, per_xcd);
  return hipGetLastError();
}

}  // namespace qattn
