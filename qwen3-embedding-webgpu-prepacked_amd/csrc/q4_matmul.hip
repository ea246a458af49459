// q4_matmul.hip -- Q4_0 "tile32-compact" dequant-GEMM: Y = X W^T with fp16 activations X [M, K]
// and 4-bit weights W [N, K]: the model's four projections (QKV, attention output, gate/up, down).
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
//     v_mfma_f32_32x32x16_f16 with fp32 accumulators (64 VGPRs); 128 VGPRs in all, so up to four
//     workgroups share a CU.  Small launches use 64 x 128 tiles (wavefronts of 32 x 64);
//   * per 32-column K block: the X tile (128 rows x 64 B) goes HBM -> LDS by LDS-DMA
//     (buffer_load ... lds, 16 B per lane); each weight record of the tile's 128 rows is read
//     once (scale word + 8 quant bytes per thread) and dequantised into a B tile in LDS: the
//     nibbles become f16 by bit-OR into 1024.0 (f16(1024 + q)), an exact subtract of 1032 and one
//     f16 multiply by the scale (the same single rounding as the reference's f16 product);
//   * both tiles are double-buffered with one barrier per K block, laid out with a 16-byte XOR
//     swizzle so the fragment reads (ds_read_b128) are conflict free; the next block's
//     fragments are read into a second register set right after the barrier, and the weight
//     records are loaded three blocks ahead (clamped past the end, so every path issues the same
//     loads and the wait counts are exact);
//   * tiles are numbered so that consecutive workgroups on one XCD (workgroup b runs on XCD
//     b % 8) walk the N tiles of one M tile: its X rows stay in that XCD's L2;
//   * the SWIGLU variant (the FFN's gate/up projection, model.ts:126-127) maps each workgroup's B
//     rows onto a feature's gate and up rows and writes silu(gate) * up instead of the projection.
//   * launches of at most kQ4DirectBlocks 32 x 32 output blocks (small M) run q4_direct_kernel
//     instead: one workgroup per block, no tile staging, the same MFMA chains per output element,
//     so its rows equal the tiled kernel's bit for bit; up to one block per CU each K chunk runs
//     in a wavefront of its own and the chains meet in LDS.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "model_ops.h"

namespace qattn {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef uint32_t u2 __attribute__((ext_vector_type(2)));
typedef uint32_t u4 __attribute__((ext_vector_type(4)));

constexpr int kQ4TileN = 128;   // workgroup tile columns; rows 64 BM (BM = 2, or 1 for small launches)
constexpr int kQ4Record = 20;   // bytes per (row, 32-column block)
// Below this many 128 x 128 tiles a launch uses 64-row workgroup tiles (twice as many
// workgroups on the 256 CUs; measured 10-11% faster for the model's output and down projections
// at M = 500-1,419, slower above about 160 tiles).  Each output element is computed the same way
// in both.
constexpr int kQ4SmallLaunch = 160;
// Fixed K split: every output element is the fp32 sum, in chunk order, of MFMA chains over
// chunks of kQ4ChunkBlocks 32-column K blocks, each chain from a zero accumulator:
// y = f16((c0 + c1) + c2) for K = 3072.  The split depends on K alone, so a row's result does
// not depend on the batch whichever way a launch computes it: in registers (every chunk in one
// workgroup, a second accumulator set) or, for launches with few tiles, one workgroup per
// (tile, chunk) writing fp32 partials that q4_reduce_kernel sums in the same order.
constexpr int kQ4ChunkBlocks = 32;
// Launches with fewer than this many 64 x 128 tiles (two per CU) and more than one chunk split
// the chunks over workgroups when the caller provides a workspace (chunks x M x N fp32).  The
// model's output and down projections split up to M = 4,095: 16 x 150 tokens forward 2.5% faster
// than with the limit at 256 tiles, the other batch sizes unchanged.
constexpr int kQ4SplitTiles = 512;

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

typedef __attribute__((address_space(3))) void lds_void_t;

// LDS tiles: 128 rows x 32 columns of fp16 (64 B per row) for X (A) and for the dequantised
// weights (B, row = output column n).  The four 16-byte chunks of row r sit at physical chunk
// c ^ ((r >> 2) & 3): 16 consecutive rows reading one logical chunk then cover all 64 banks, so
// the fragment reads (lanes 0-15 / 16-31 / ... take 16 consecutive rows) are conflict free.
__device__ inline uint32_t q4_lds_off(int row, int chunk) { return row * 64 + ((chunk ^ ((row >> 2) & 3)) << 4); }

// The memory and matrix builtins behind plain (non-template) device functions: the kernel uses
// them in BM-dependent loops, and hipcc's host pass drops a kernel template's host stub when
// such a builtin sits in a dependent context.
__device__ inline void q4_dma16(__amdgpu_buffer_rsrc_t rs, char* dst, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)dst, 16, off, 0, 0, 0);
}
__device__ inline void q4_store_b16(_Float16 v, __amdgpu_buffer_rsrc_t rs, uint32_t off) {
  __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(unsigned short, v), rs, off, 0, 0);
}
__device__ inline f16x q4_mfma(h8 a, h8 b, f16x c) { return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0); }

// SWIGLU: the weight is [gate (N/2 rows) | up (N/2 rows)] and the output is silu(gate) * up, N/2
// columns: the workgroup of tile column tn takes gate rows 64 tn .. +63 and the matching up rows
// (B rows 0-31 gate, 32-63 up, 64-95 gate, 96-127 up), so every wave holds the gate and up
// accumulators of the same 32 features in the same lanes and applies swiglu_value to them.
// CH = 0: K within one chunk (one chain); 1: every chunk in this workgroup (a second set of
// accumulators holds the finished chunks' sum); 2: one chunk per workgroup (work unit t =
// tile * chunks + chunk), its chain stored as fp32 to part[chunk][m][n].
template <bool SWIGLU, int BM, int CH>
__global__ __launch_bounds__(256, 2) void q4_matmul_kernel(const _Float16* __restrict__ x, int64_t ldx, int M, int K,
                                                           const uint8_t* __restrict__ w, uint32_t w_bytes, int N,
                                                           _Float16* __restrict__ y, int64_t ldy, int tiles_n,
                                                           int tiles_total, int per_xcd, float* __restrict__ part,
                                                           int chunks) {
  // Double-buffered A and B tiles: four distinct objects, each buffer choice fixed at compile
  // time, so the compiler sees that LDS-DMA writes in flight never alias the tile being read.
  constexpr int kTileM = 64 * BM;
  __shared__ __attribute__((aligned(1024))) char sA0[kTileM * 64];
  __shared__ __attribute__((aligned(1024))) char sA1[kTileM * 64];
  __shared__ __attribute__((aligned(1024))) char sB0[kQ4TileN * 64];
  __shared__ __attribute__((aligned(1024))) char sB1[kQ4TileN * 64];

  // Tile of this workgroup: XCD b % 8 owns tiles [xcd * per_xcd, (xcd + 1) * per_xcd).
  const int b = blockIdx.x;
  const int u = (b & 7) * per_xcd + (b >> 3);
  if (u >= tiles_total) return;
  const int t = CH == 2 ? u / chunks : u;
  const int m0 = (t / tiles_n) * kTileM, n0 = (t % tiles_n) * kQ4TileN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hl = lane >> 5;
  const int wr = 32 * BM * (wave & 1), wc = 64 * (wave >> 1);  // this wave's 32 BM x 64 inside the tile
  const int kblocks = K >> 5;
  // K blocks of this workgroup: all of them, or (CH == 2) one chunk.
  const int kb_first = CH == 2 ? (u % chunks) * kQ4ChunkBlocks : 0;
  const int kb_end = CH == 2 ? min(kb_first + kQ4ChunkBlocks, kblocks) : kblocks;

  const auto xrs = q4_rsrc(x, (uint32_t)M * (uint32_t)ldx * 2u);  // rows >= M read as zeros
  const auto wrs = q4_rsrc(w, w_bytes);
  const auto yrs = q4_rsrc(y, (uint32_t)M * (uint32_t)ldy * 2u);

  // ---- A: LDS-DMA, 16 B per lane per instruction, 1 KiB (16 rows) per wave instruction.
  // Instruction j of wave `wave` fills rows 16 (BM wave + j) .. +15; lane's LDS slot p = lane * 16
  // within that KiB is row 16 (BM wave + j) + lane / 4, physical chunk lane & 3, which holds
  // logical chunk (lane & 3) ^ ((row >> 2) & 3): columns 8 * that .. +7 of the K block.
  uint32_t a_src[BM];
#pragma unroll
  for (int j = 0; j < BM; ++j) {
    const int row = 16 * (BM * wave + j) + (lane >> 2);
    const int chunk = (lane & 3) ^ ((row >> 2) & 3);
    a_src[j] = (uint32_t)(m0 + row) * (uint32_t)ldx * 2u + 16u * chunk;
  }
  auto load_a = [&](char* dst, int kb) {
    kb = kb < kb_end ? kb : kb_end - 1;  // past the end: re-read the last block (never used)
#pragma unroll
    for (int j = 0; j < BM; ++j) q4_dma16(xrs, dst + 1024 * (BM * wave + j), a_src[j] + (uint32_t)kb * 64u);
  };

  // ---- B: thread (row n = tid / 2, half h = tid & 1) owns quant bytes 8h .. 8h+7 of the record
  // of (n0 + n, kb): their low nibbles are columns 8h .. +7 (chunk h), their high nibbles columns
  // 16 + 8h .. +7 (chunk 2 + h).  Records of rows past the tensor read as zeros.
  const int brow = tid >> 1, bhalf = tid & 1;
  const int wtile = SWIGLU ? ((brow >> 5) & 1 ? N >> 6 : 0) + (n0 >> 6) + (brow >> 6) : (n0 + brow) >> 5;
  const uint32_t w_rec = ((uint32_t)wtile * (uint32_t)kblocks * 32u + (uint32_t)(brow & 31)) * kQ4Record;
  const uint32_t w_step = 32u * kQ4Record;
  const uint32_t b_lo = q4_lds_off(brow, bhalf), b_hi = q4_lds_off(brow, 2 + bhalf);
  struct WRegs {
    uint32_t scale;
    u2 q;
  };
  auto load_w = [&](WRegs& r, int kb) {
    kb = kb < kb_end ? kb : kb_end - 1;
    const uint32_t off = w_rec + (uint32_t)kb * w_step;
    r.scale = __builtin_amdgcn_raw_buffer_load_b32(wrs, off, 0, 0);
    r.q = __builtin_amdgcn_raw_buffer_load_b64(wrs, off + 4u + 8u * bhalf, 0, 0);
  };
  auto store_b = [&](char* dst, const WRegs& r) {
    const _Float16 s = __builtin_bit_cast(h2, r.scale)[0];
    const h2 scale = {s, s};
    *reinterpret_cast<h8*>(dst + b_lo) = dequant8<false>(r.q, scale);
    *reinterpret_cast<h8*>(dst + b_hi) = dequant8<true>(r.q, scale);
  };

  // ---- fragments: lane reads row (wr or wc) + 32 blk + l32, logical chunk 2 s + hl.
  f16x acc[BM][2];
#pragma unroll
  for (int mb = 0; mb < BM; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = f16x{};
  // Fragments of one K block: two sets, alternating by block parity, so the next block's reads
  // are in flight while this block's MFMAs run.
  struct Frags {
    h8 a[BM][2], b[2][2];
  };
  Frags frag[2];
  auto read_frags = [&](const char* a_t, const char* b_t, Frags& f) {
#pragma unroll
    for (int blk = 0; blk < 2; ++blk)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        if (blk < BM) f.a[blk][s] = *reinterpret_cast<const h8*>(a_t + q4_lds_off(wr + 32 * blk + l32, 2 * s + hl));
        f.b[blk][s] = *reinterpret_cast<const h8*>(b_t + q4_lds_off(wc + 32 * blk + l32, 2 * s + hl));
      }
  };
  // The MFMA order of an output block -- s, then its K blocks in turn -- is the same for BM = 1
  // and 2, so rows do not depend on the tile height a launch picks.
  // fresh: the first K block of a chain (CH == 1 chunks after the first): step 0 accumulates onto
  // the inline constant 0, which is what the zeroed accumulators would add.
  auto mma = [&](const Frags& f, auto fresh) {
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int mb = 0; mb < BM; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
          acc[mb][nb] = q4_mfma(f.a[mb][s], f.b[nb][s], decltype(fresh)::value && s == 0 ? f16x{} : acc[mb][nb]);
  };

  // ---- pipeline.  Step kb (P = kb & 1, compile time): issue A(kb+1) into sA<1-P> and W(kb+3)
  // into register stage (kb+3) % 4; dequantise W(kb+1) (loaded two steps ago) into sB<1-P>; run
  // block kb's MFMAs on the fragments read at the end of the previous step; wait for A(kb+1)
  // (only W(kb+3), issued after it, may still be in flight: vmcnt(2)); barrier; read block
  // kb+1's fragments.  sB<1-P> is free at its write: its last reads (block kb-1's fragments)
  // were consumed by MFMAs before the previous barrier.  Every load is issued (clamped past the
  // end), so the counts are the same on every path.
  WRegs wreg[4];
  load_a(sA0, kb_first);
  load_w(wreg[0], kb_first);
  load_w(wreg[1], kb_first + 1);
  load_w(wreg[2], kb_first + 2);
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8) | 4);  // vmcnt(4): A(0), W(0) landed
  store_b(sB0, wreg[0]);
  __syncthreads();
  read_frags(sA0, sB0, frag[0]);
  auto step = [&](auto pconst, auto wcur, auto wnext, int kb, auto fresh) {
    constexpr int P = decltype(pconst)::value;
    constexpr int WN = decltype(wnext)::value;   // stage of W(kb+1)
    constexpr int WA = decltype(wcur)::value;    // stage receiving W(kb+3)
    char* const a_nxt = P == 0 ? sA1 : sA0;
    char* const b_nxt = P == 0 ? sB1 : sB0;
    load_a(a_nxt, kb + 1);
    load_w(wreg[WA], kb + 3);
    store_b(b_nxt, wreg[WN]);
    if (kb < kb_end) mma(frag[P], fresh);
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8) | 2);  // vmcnt(2)
    __syncthreads();
    read_frags(a_nxt, b_nxt, frag[1 - P]);
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;
  using I2 = std::integral_constant<int, 2>;
  using I3 = std::integral_constant<int, 3>;
  // Chunks of kQ4ChunkBlocks (a multiple of the 4-step group, so the steps' compile-time
  // buffer and register-stage choices follow from kb as before); CH == 1 folds each finished
  // chunk into tot and starts the next chain from zero.
  using Fresh = std::integral_constant<bool, true>;
  using Cont = std::integral_constant<bool, false>;
  auto four_steps = [&](int kb, auto fresh) {
    step(I0{}, I3{}, I1{}, kb, fresh);
    step(I1{}, I0{}, I2{}, kb + 1, Cont{});
    step(I0{}, I1{}, I3{}, kb + 2, Cont{});
    step(I1{}, I2{}, I0{}, kb + 3, Cont{});
  };
  f16x tot[CH == 1 ? BM : 1][2];
  if constexpr (CH == 1) {
    // Chunk 0 into acc, copied to tot; every later chunk a fresh chain in acc, added to tot.
    for (int kb = 0; kb < kQ4ChunkBlocks; kb += 4) four_steps(kb, Cont{});
#pragma unroll
    for (int mb = 0; mb < BM; ++mb)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) tot[mb][nb] = acc[mb][nb];
    for (int c0 = kQ4ChunkBlocks; c0 < kblocks; c0 += kQ4ChunkBlocks) {
      const int c1 = min(c0 + kQ4ChunkBlocks, kblocks);
      four_steps(c0, Fresh{});
      for (int kb = c0 + 4; kb < c1; kb += 4) four_steps(kb, Cont{});
#pragma unroll
      for (int mb = 0; mb < BM; ++mb)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) tot[mb][nb] = tot[mb][nb] + acc[mb][nb];
    }
  } else {
    for (int kb = kb_first; kb < kb_end; kb += 4) four_steps(kb, Cont{});
  }
  __builtin_amdgcn_s_waitcnt(0);  // the clamped loads past the end land before the LDS is released
  if constexpr (CH == 1) {
#pragma unroll
    for (int mb = 0; mb < BM; ++mb)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) acc[mb][nb] = tot[mb][nb];
  }

  // D (32 x 32 per block): lane holds column l32 and rows 8 (r / 4) + 4 hl + r % 4, r = 0..15.
  // Columns >= N are skipped here; rows >= M fall outside the Y resource and are dropped.
  const int wm = m0 + wr, wn = n0 + wc;
  if constexpr (CH == 2) {
    // This chunk's chains, fp32, to part[chunk][m][n] (rows >= M and columns >= N skipped).
    float* const pc = part + (size_t)(u % chunks) * (size_t)M * (size_t)N;
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int n = wn + 32 * nb + l32;
      if (n < N) {
#pragma unroll
        for (int mb = 0; mb < BM; ++mb)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int m = wm + 32 * mb + 8 * (r >> 2) + 4 * hl + (r & 3);
            if (m < M) pc[(size_t)m * N + n] = acc[mb][nb][r];
          }
      }
    }
    return;
  }
  if constexpr (SWIGLU) {
    // Block nb = 0 holds gate, nb = 1 up, of output features (n0 + wc) / 2 + l32.
    const uint32_t n = (uint32_t)((wn >> 1) + l32);
#pragma unroll
    for (int mb = 0; mb < BM; ++mb)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = wm + 32 * mb + 8 * (r >> 2) + 4 * hl + (r & 3);
        const uint32_t off = m < M ? ((uint32_t)m * (uint32_t)ldy + n) * 2u : 0x80000000u;
        q4_store_b16(swiglu_value((_Float16)acc[mb][0][r], (_Float16)acc[mb][1][r]), yrs, off);
      }
    return;
  }
#pragma unroll
  for (int nb = 0; nb < 2; ++nb) {
    const int n = wn + 32 * nb + l32;
    if (n < N) {
#pragma unroll
      for (int mb = 0; mb < BM; ++mb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int m = wm + 32 * mb + 8 * (r >> 2) + 4 * hl + (r & 3);
          const uint32_t off = m < M ? ((uint32_t)m * (uint32_t)ldy + (uint32_t)n) * 2u : 0x80000000u;
          q4_store_b16((_Float16)acc[mb][nb][r], yrs, off);
        }
    }
  }
}

// ---- small launches (at most kQ4DirectBlocks 32 x 32 output blocks): one wavefront per block,
// one wavefront per workgroup, and no LDS.
// At small M the tiled kernel's time is its K loop's latency chain -- dequantised weights to
// LDS, barrier, fragment reads, MFMAs -- about 0.3 us per 32-column K block for every M up to
// ~1,500, on as few as 8 workgroups.  Here each wavefront loads its own X rows and weight records
// straight into MFMA fragment registers, kQ4Ahead K blocks ahead, dequantises them with the same
// code and runs the same MFMA chain: per output element the same operands in the same order
// (K block by K block, its 16-column step 0 then step 1, from a zero accumulator), so the result
// is bit for bit the tiled kernel's and a row does not depend on the batch it is in.
// Lane (l32, hl) holds X row m0 + l32 and weight row n0 + l32, columns 16 s + 8 hl .. +7 of the
// K block in step s (the tiled kernel's fragment layout).  SWIGLU: two chains, the gate rows
// n0 + l32 and the up rows n_inter + n0 + l32 of the 32 output features n0 .. n0 + 31.
// A wavefront is bound by its own dequantisation VALU work (~0.11 us per K block, twice that
// with SWIGLU's two chains) and its X loads, which touch one cache line per row: one wavefront
// per workgroup spreads the blocks over as many CUs (measured 2x faster than four per
// workgroup).  Up to 512 blocks (two per CU) it beats the tiled kernel on all four projection
// shapes; deeper rings and coalesced X loads staged through LDS measured slower.
constexpr int kQ4DirectBlocks = 512;
constexpr int kQ4Ahead = 8;  // K blocks in flight per wavefront (a ring of register stages)

// One workgroup per output block.  CH = 0: K is one chunk.  CH = 1: one wavefront per K chunk;
// wavefront c runs chunk c's chain, the chains meet in LDS and wavefront 0 sums them in chunk
// order, as the tiled kernel does.  CH = 2: one wavefront runs the chunks in turn and folds each
// finished chain into a second accumulator (launches whose chunk wavefronts would crowd the CUs).
// CH = 3 (SWIGLU, K one chunk): two wavefronts, the gate chain and the up chain, which meet in LDS
// for the epilogue.
constexpr int kQ4MaxChunks = 8;  // K <= 8192 on this path
// CH = 1 up to one output block per CU.  Measured at M = 15-240 for the output and down
// projections: 25-46% faster than one wavefront folding the chunks; with more blocks the chunk
// wavefronts share CUs and were up to 13% slower.
constexpr int kQ4ChunkParallelBlocks = 256;
template <bool SWIGLU, int CH>
__global__ __launch_bounds__(CH == 1 ? 64 * kQ4MaxChunks : CH == 3 ? 128 : 64) void q4_direct_kernel(
    const _Float16* __restrict__ x, int64_t ldx, int M, int K, const uint8_t* __restrict__ w, uint32_t w_bytes, int N,
    _Float16* __restrict__ y, int64_t ldy, int blocks_m, int blocks_total) {
  static_assert(CH != 3 || SWIGLU, "gate/up wavefront pairs are a SWIGLU form");
  const int lane = threadIdx.x & 63, l32 = lane & 31, hl = lane >> 5;
  constexpr bool CHUNKED = CH == 1;
  constexpr bool PAIR = CH == 3;          // this wavefront runs one of the two SWIGLU chains
  constexpr bool BOTH = SWIGLU && !PAIR;  // this wavefront runs the gate and the up chain
  const int half = PAIR ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : 0;  // 0 gate, 1 up
  const int chunk = CHUNKED ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) : 0;
  // block g: the M blocks of one N block are consecutive (they share weight records in L2)
  const int g = blockIdx.x;
  if (g >= blocks_total) return;  // the whole workgroup: its barrier below stays uniform
  const int m0 = (g % blocks_m) * 32, n0 = (g / blocks_m) * 32;
  const int kblocks_all = K >> 5;
  // This wavefront's K blocks [kb0, kblocks): one chunk, or all of K.
  const int kb0 = CHUNKED ? chunk * kQ4ChunkBlocks : 0;
  const int kblocks = CHUNKED ? min(kb0 + kQ4ChunkBlocks, kblocks_all) : kblocks_all;
  const int n_out = SWIGLU ? N >> 1 : N;  // output columns

  const auto xrs = q4_rsrc(x, (uint32_t)M * (uint32_t)ldx * 2u);  // rows >= M read as zeros
  const auto wrs = q4_rsrc(w, w_bytes);                          // rows >= N read as zeros
  const auto yrs = q4_rsrc(y, (uint32_t)M * (uint32_t)ldy * 2u);
  const uint32_t x_row = (uint32_t)(m0 + l32) * (uint32_t)ldx * 2u + 16u * hl;
  auto w_rec = [&](int n) {
    return ((uint32_t)(n >> 5) * (uint32_t)kblocks_all * 32u + (uint32_t)(n & 31)) * kQ4Record;
  };
  const uint32_t wu_rec = SWIGLU ? w_rec(n_out + n0 + l32) : 0u;
  // The first chain's records: the gate rows (the up rows for the second wavefront of a pair).
  const uint32_t wg_rec = PAIR && half ? wu_rec : w_rec(n0 + l32);
  const uint32_t w_step = 32u * kQ4Record;

  struct Stage {
    h8 a[2];
    uint32_t sg, su;
    u2 qg, qu;
  };
  constexpr int kOps = BOTH ? 6 : 4;  // vector-memory instructions per K block
  auto load = [&](Stage& st, int kb) {
    kb = kb < kblocks ? kb : kblocks - 1;  // past the end: re-read the last block (never used)
    const uint32_t xo = x_row + (uint32_t)kb * 64u;
    st.a[0] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(xrs, xo, 0, 0));
    st.a[1] = __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(xrs, xo + 32u, 0, 0));
    const uint32_t go = wg_rec + (uint32_t)kb * w_step;
    st.sg = __builtin_amdgcn_raw_buffer_load_b32(wrs, go, 0, 0);
    st.qg = __builtin_amdgcn_raw_buffer_load_b64(wrs, go + 4u + 8u * hl, 0, 0);
    if constexpr (BOTH) {
      const uint32_t uo = wu_rec + (uint32_t)kb * w_step;
      st.su = __builtin_amdgcn_raw_buffer_load_b32(wrs, uo, 0, 0);
      st.qu = __builtin_amdgcn_raw_buffer_load_b64(wrs, uo + 4u + 8u * hl, 0, 0);
    }
  };
  f16x acc_g = {}, acc_u = {};
  auto mma = [&](const Stage& st) {
    const _Float16 sg = __builtin_bit_cast(h2, st.sg)[0];
    const h2 scale_g = {sg, sg};
    acc_g = q4_mfma(st.a[0], dequant8<false>(st.qg, scale_g), acc_g);
    acc_g = q4_mfma(st.a[1], dequant8<true>(st.qg, scale_g), acc_g);
    if constexpr (BOTH) {
      const _Float16 su = __builtin_bit_cast(h2, st.su)[0];
      const h2 scale_u = {su, su};
      acc_u = q4_mfma(st.a[0], dequant8<false>(st.qu, scale_u), acc_u);
      acc_u = q4_mfma(st.a[1], dequant8<true>(st.qu, scale_u), acc_u);
    }
  };
  Stage ring[kQ4Ahead];
  // The waits count loads in issue order: the compiler must not move them across blocks.
#pragma unroll
  for (int j = 0; j < kQ4Ahead; ++j) {
    load(ring[j], kb0 + j);
    __builtin_amdgcn_sched_barrier(0);
  }
  // Block kb sits in stage kb % kQ4Ahead; the loads of the kQ4Ahead - 1 blocks after it may still
  // be in flight when it is used (loads retire in issue order), then its stage takes block
  // kb + kQ4Ahead.
  constexpr int kWait = (kQ4Ahead - 1) * kOps;
  static_assert(kWait < 64, "vmcnt is 6 bits");
  static_assert(kQ4ChunkBlocks % kQ4Ahead == 0, "chunk ends fall between ring passes");
  f16x tot_g = {}, tot_u = {};
  for (int kb = kb0; kb < kblocks; kb += kQ4Ahead) {
#pragma unroll
    for (int j = 0; j < kQ4Ahead; ++j) {
      __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8) | (kWait & 15) | ((kWait >> 4) << 14));
      if (kb + j < kblocks) mma(ring[j]);
      __builtin_amdgcn_sched_barrier(0);
      load(ring[j], kb + j + kQ4Ahead);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (CH == 2) {
      // End of a chunk (or of K): fold the chain into the sum and start the next from zero.
      if ((kb + kQ4Ahead) % kQ4ChunkBlocks == 0 || kb + kQ4Ahead >= kblocks) {
        tot_g = kb < kQ4ChunkBlocks ? acc_g : tot_g + acc_g;
        acc_g = f16x{};
        if constexpr (BOTH) {
          tot_u = kb < kQ4ChunkBlocks ? acc_u : tot_u + acc_u;
          acc_u = f16x{};
        }
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  if constexpr (CH == 2) {
    acc_g = tot_g;
    acc_u = tot_u;
  }
  if constexpr (CHUNKED) {
    // The chains of chunks 1.. meet wavefront 0's (chunk 0) in LDS; it adds them in chunk order.
    __shared__ f16x part_g[kQ4MaxChunks - 1][64];
    __shared__ f16x part_u[SWIGLU ? kQ4MaxChunks - 1 : 1][SWIGLU ? 64 : 1];
    const int nch = (kblocks_all + kQ4ChunkBlocks - 1) / kQ4ChunkBlocks;
    if (chunk > 0) {
      part_g[chunk - 1][lane] = acc_g;
      if constexpr (SWIGLU) part_u[chunk - 1][lane] = acc_u;
    }
    __syncthreads();
    if (chunk > 0) return;
    for (int c = 1; c < nch; ++c) {
      acc_g = acc_g + part_g[c - 1][lane];
      if constexpr (SWIGLU) acc_u = acc_u + part_u[c - 1][lane];
    }
  }
  if constexpr (PAIR) {
    __shared__ f16x up[64];
    if (half) up[lane] = acc_g;
    __syncthreads();
    if (half) return;
    acc_u = up[lane];
  }

  // D (32 x 32): lane holds column l32 and rows 8 (r / 4) + 4 hl + r % 4 -- as the tiled kernel.
  const int n = n0 + l32;
  if (n >= n_out) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int m = m0 + 8 * (r >> 2) + 4 * hl + (r & 3);
    const uint32_t off = m < M ? ((uint32_t)m * (uint32_t)ldy + (uint32_t)n) * 2u : 0x80000000u;
    if constexpr (SWIGLU)
      q4_store_b16(swiglu_value((_Float16)acc_g[r], (_Float16)acc_u[r]), yrs, off);
    else
      q4_store_b16((_Float16)acc_g[r], yrs, off);
  }
}

template <bool SWIGLU>
void launch_q4_direct(const _Float16* x, int64_t ldx, int M, int K, const uint8_t* w, uint32_t w_bytes, int N,
                      _Float16* y, int64_t ldy, hipStream_t stream) {
  const int n_out = SWIGLU ? N / 2 : N;
  const int blocks_m = (M + 31) / 32, blocks = blocks_m * ((n_out + 31) / 32);
  const int chunks = (K / 32 + kQ4ChunkBlocks - 1) / kQ4ChunkBlocks;
  if (chunks > 1 && blocks <= kQ4ChunkParallelBlocks)
    hipLaunchKernelGGL((q4_direct_kernel<SWIGLU, 1>), dim3((unsigned)blocks), dim3(64 * chunks), 0, stream, x, ldx,
                       M, K, w, w_bytes, N, y, ldy, blocks_m, blocks);
  else if (chunks > 1)
    hipLaunchKernelGGL((q4_direct_kernel<SWIGLU, 2>), dim3((unsigned)blocks), dim3(64), 0, stream, x, ldx, M, K, w,
                       w_bytes, N, y, ldy, blocks_m, blocks);
  else if (SWIGLU && blocks <= kQ4ChunkParallelBlocks)
    hipLaunchKernelGGL((q4_direct_kernel<SWIGLU, SWIGLU ? 3 : 0>), dim3((unsigned)blocks), dim3(128), 0, stream, x,
                       ldx, M, K, w, w_bytes, N, y, ldy, blocks_m, blocks);
  else
    hipLaunchKernelGGL((q4_direct_kernel<SWIGLU, 0>), dim3((unsigned)blocks), dim3(64), 0, stream, x, ldx, M,
                       K, w, w_bytes, N, y, ldy, blocks_m, blocks);
}

// y = f16(part[0] + part[1] + ...), summed in chunk order (part: chunks x M x N fp32).  Thread =
// four consecutive columns of row blockIdx.y (16-byte partial loads and an 8-byte store when the
// alignment allows; the same fp32 additions either way).
__global__ __launch_bounds__(256) void q4_reduce_kernel(const float* __restrict__ part, int chunks, int M, int N,
                                                        _Float16* __restrict__ y, int64_t ldy) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  const int m = blockIdx.y;
  const int n0 = (blockIdx.x * 256 + threadIdx.x) * 4;
  if (n0 >= N) return;
  const size_t plane = (size_t)M * (size_t)N;
  const float* p = part + (size_t)m * N + n0;
  _Float16* yr = y + (int64_t)m * ldy + n0;
  if ((N & 3) == 0) {  // rows, planes and this thread's columns start 16-byte aligned
    f4 s = *reinterpret_cast<const f4*>(p);
    for (int c = 1; c < chunks; ++c) s = s + *reinterpret_cast<const f4*>(p + (size_t)c * plane);
    const h4 v = {(_Float16)s[0], (_Float16)s[1], (_Float16)s[2], (_Float16)s[3]};
    if ((reinterpret_cast<uintptr_t>(yr) & 7) == 0) {
      *reinterpret_cast<h4*>(yr) = v;
    } else {
      yr[0] = v[0];
      yr[1] = v[1];
      yr[2] = v[2];
      yr[3] = v[3];
    }
  } else {
    for (int j = 0; j < 4 && n0 + j < N; ++j) {
      float s = p[j];
      for (int c = 1; c < chunks; ++c) s = s + p[(size_t)c * plane + j];
      yr[j] = (_Float16)s;
    }
  }
}

// Grid: 8 * ceil(tiles / 8) workgroups of 256 threads (the surplus ones exit at once), 128 x 128
// tiles, or 64 x 128 when the launch has fewer than kQ4SmallLaunch 128 x 128 tiles.
template <bool SWIGLU, int BM, int CH>
void launch_q4_shape(const _Float16* x, int64_t ldx, int M, int K, const uint8_t* w, uint32_t w_bytes, int N,
                     _Float16* y, int64_t ldy, hipStream_t stream, float* part = nullptr, int chunks = 1) {
  const int tiles_m = (M + 64 * BM - 1) / (64 * BM), tiles_n = (N + kQ4TileN - 1) / kQ4TileN;
  const int units = tiles_m * tiles_n * (CH == 2 ? chunks : 1), per_xcd = (units + 7) / 8;
  hipLaunchKernelGGL((q4_matmul_kernel<SWIGLU, BM, CH>), dim3((unsigned)(8 * per_xcd)), dim3(256), 0, stream, x, ldx,
                     M, K, w, w_bytes, N, y, ldy, tiles_n, units, per_xcd, part, chunks);
}
template <bool SWIGLU, int BM>
void launch_q4_tiled(const _Float16* x, int64_t ldx, int M, int K, const uint8_t* w, uint32_t w_bytes, int N,
                     _Float16* y, int64_t ldy, hipStream_t stream) {
  if (K / 32 > kQ4ChunkBlocks)
    launch_q4_shape<SWIGLU, BM, 1>(x, ldx, M, K, w, w_bytes, N, y, ldy, stream);
  else
    launch_q4_shape<SWIGLU, BM, 0>(x, ldx, M, K, w, w_bytes, N, y, ldy, stream);
}

size_t q4_split_bytes(int M, int K, int N) {
  const int chunks = (K / 32 + kQ4ChunkBlocks - 1) / kQ4ChunkBlocks;
  const int64_t tiles = (int64_t)((M + 63) / 64) * ((N + kQ4TileN - 1) / kQ4TileN);
  if (chunks < 2 || tiles >= kQ4SplitTiles) return 0;
  return (size_t)chunks * (size_t)M * (size_t)N * sizeof(float);
}

template <bool SWIGLU>
hipError_t launch_q4(const _Float16* x, int64_t ldx, int M, int K, const uint8_t* w, uint32_t w_bytes, int N,
                     _Float16* y, int64_t ldy, hipStream_t stream, float* ws, size_t ws_bytes,
                     const RowNorm* norm = nullptr, bool* normed = nullptr) {
  const int64_t big_tiles = (int64_t)((M + 127) / 128) * ((N + kQ4TileN - 1) / kQ4TileN);
  const int n_out = SWIGLU ? N / 2 : N;
  const size_t split = SWIGLU ? 0 : q4_split_bytes(M, K, N);
  const int chunks = (K / 32 + kQ4ChunkBlocks - 1) / kQ4ChunkBlocks;
  if ((int64_t)((M + 31) / 32) * ((n_out + 31) / 32) <= kQ4DirectBlocks && chunks <= kQ4MaxChunks) {
    launch_q4_direct<SWIGLU>(x, ldx, M, K, w, w_bytes, N, y, ldy, stream);
  } else if (split && ws && split <= ws_bytes) {
    launch_q4_shape<SWIGLU, 1, 2>(x, ldx, M, K, w, w_bytes, N, y, ldy, stream, ws, chunks);
    if (norm && N % 8 == 0 && N <= kRmsMaxWidth) {
      // the sums go straight into the residual add + RMSNorm that follows the projection
      const hipError_t e = launch_reduce_rmsnorm(ws, chunks, M, N, *norm, stream);
      if (e != hipSuccess) return e;
      if (normed) *normed = true;
    } else {
      // one row per grid row (M < 64 * kQ4SplitTiles here), 1024 columns per workgroup
      hipLaunchKernelGGL(q4_reduce_kernel, dim3((unsigned)((N + 1023) / 1024), (unsigned)M), dim3(256), 0, stream,
                         ws, chunks, M, N, y, ldy);
    }
  } else if (big_tiles < kQ4SmallLaunch) {
    launch_q4_tiled<SWIGLU, 1>(x, ldx, M, K, w, w_bytes, N, y, ldy, stream);
  } else {
    launch_q4_tiled<SWIGLU, 2>(x, ldx, M, K, w, w_bytes, N, y, ldy, stream);
  }
  return hipGetLastError();
}

hipError_t launch_q4_matmul(const _Float16* x, int64_t ldx, int M, int K, const uint8_t* w, uint32_t w_bytes, int N,
                            _Float16* y, int64_t ldy, hipStream_t stream, float* ws, size_t ws_bytes,
                            const RowNorm* norm, bool* normed) {
  if (M <= 0 || N <= 0) return hipSuccess;
  return launch_q4<false>(x, ldx, M, K, w, w_bytes, N, y, ldy, stream, ws, ws_bytes, norm, normed);
}

// y [M, n_inter] = swiglu of the [gate | up] projection; the weight has 2 n_inter rows and
// n_inter is a multiple of 64.
hipError_t launch_q4_matmul_swiglu(const _Float16* x, int64_t ldx, int M, int K, const uint8_t* w, uint32_t w_bytes,
                                   int n_inter, _Float16* y, int64_t ldy, hipStream_t stream) {
  if (M <= 0 || n_inter <= 0) return hipSuccess;
  return launch_q4<true>(x, ldx, M, K, w, w_bytes, 2 * n_inter, y, ldy, stream, nullptr, 0);
}

}  // namespace qattn
