// tile_body_bench.hip -- tile-body microbenchmark for the attention kernel's schedule choices.
//
// Runs the attention kernel's per-tile work (the work that replaces the reference's hot loop,
// src/webgpu/ops.ts:194-240; csrc/attn_fwd.hip: S^T = K Q^T on
// v_mfma_f32_32x32x16_f16 with K fragments from swizzled LDS, the lazy-max softmax with fp16
// probabilities and v_fma_mix row sums, O^T += V^T P^T with ds_read_b64_tr_b16 V fragments) over
// tiles that stay in LDS: no global memory traffic, no work items, no hand-over.  It bounds what
// a schedule of that work can reach on the matrix cores, and compares schedules:
//   MODE 0  the kernel's pipelined body: S(j+1), PV(j-1) and softmax(j) per iteration, two score /
//           probability register sets, 64 KiB of LDS, 2 workgroups (2 waves per SIMD) per CU;
//   MODE 1  serial 64-key tiles (S, softmax, PV; one register set, two barriers per tile),
//           at most 168 VGPRs, 48 KiB of LDS: 3 workgroups per CU;
//   MODE 2  serial 32-key half steps (one 16-register score set), 3 workgroups per CU.
// Usage: tile_body_bench MODE NTILES WORKGROUPS_PER_CU
// Prints the time per tile-step and the FLOP rate: per workgroup and tile, 4 wavefronts x
// 32 rows x 64 keys x 128 dims x 2 (QK^T and PV) x 2 FLOPs.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <stdint.h>

#include <type_traits>

typedef _Float16 half_t;
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef short s4 __attribute__((ext_vector_type(4)));
typedef float f16x __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) s4 lds_s4_t;

constexpr int kRowBytes = 256;
constexpr float kLazyLimit = 32768.f;

__device__ inline f16x mfma32(h8 a, h8 b, f16x c) { return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0); }
__device__ inline float pair_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

template <int MODE>
__global__ __launch_bounds__(256, MODE == 0 ? 2 : 3) void mb(const h8* __restrict__ qin, float* __restrict__ out,
                                                              int ntiles, float c) {
  __shared__ __attribute__((aligned(1024))) char sK0[16384];
  __shared__ __attribute__((aligned(1024))) char sK1[16384];
  __shared__ __attribute__((aligned(1024))) char sV0[16384];
  __shared__ __attribute__((aligned(1024))) char sV1[MODE == 0 ? 16384 : 16];
  const int tid = threadIdx.x, lane = tid & 63, lq = lane & 31, hl = lane >> 5;
  // LDS contents: small fp16 values (the scores stay small, so the softmax keeps its fast path)
  for (int i = tid; i < 16384 / 2; i += 256) {
    const half_t v = (half_t)(((i * 37) % 17 - 8) * 0.01f);
    ((half_t*)sK0)[i] = v;
    ((half_t*)sK1)[i] = -v;
    ((half_t*)sV0)[i] = v;
    if (MODE == 0) ((half_t*)sV1)[i] = v;
  }
  __syncthreads();
  h8 qreg[8];
#pragma unroll
  for (int st = 0; st < 8; ++st) qreg[st] = qin[(blockIdx.x * 256 + tid) * 8 + st];

  const uint32_t kread_base = lq * kRowBytes + (((hl ^ lq) & 1) << 4);
  const uint32_t kread_xor = ((lq & 15) >> 1) << 5;
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
  // S^T for keys 32 half .. +31 (one block of the tile) into s
  auto qk_half = [&](const char* kt, f16x& s, int half) {
    uint32_t kx = kread_xor;
    asm volatile("" : "+v"(kx));
    auto frag = [&](int st) { return *reinterpret_cast<const h8*>(kt + kread_base + (((uint32_t)st << 5) ^ kx) + half * 32 * kRowBytes); };
    h8 a = frag(0);
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      h8 n = a;
      if (st < 7) n = frag(st + 1);
      s = mfma32(a, qreg[st], st == 0 ? f16x{} : s);
      a = n;
    }
  };
  auto qk = [&](const char* kt, f16x (&s)[2]) {
    uint32_t kx = kread_xor;
    asm volatile("" : "+v"(kx));
    auto frag = [&](int st, int half) { return *reinterpret_cast<const h8*>(kt + kread_base + (((uint32_t)st << 5) ^ kx) + half * 32 * kRowBytes); };
    h8 a0 = frag(0, 0), a1 = frag(0, 1);
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      h8 n0 = a0, n1 = a1;
      if (st < 7) {
        n0 = frag(st + 1, 0);
        n1 = frag(st + 1, 1);
      }
      s[0] = mfma32(a0, qreg[st], st == 0 ? f16x{} : s[0]);
      s[1] = mfma32(a1, qreg[st], st == 0 ? f16x{} : s[1]);
      a0 = n0;
      a1 = n1;
    }
  };
  f16x o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db] = f16x{};
  // PV over key steps t0..t1-1 (16 keys each)
  auto pv = [&](const char* vt, const h8* pf, int t0, int t1) {
#pragma unroll
    for (int t = t0; t < t1; ++t) {
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const char* vp = vt + vread[db] + t * 4096;
        const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4_t*)vp);
        const s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4_t*)(vp + 2048));
        const h4 lo_h = __builtin_bit_cast(h4, lo), hi_h = __builtin_bit_cast(h4, hi);
        const h8 va = {lo_h[0], lo_h[1], lo_h[2], lo_h[3], hi_h[0], hi_h[1], hi_h[2], hi_h[3]};
        o[db] = mfma32(va, pf[t - t0], o[db]);
      }
    }
  };
  float m_run = 0.f, l_run = 0.f;
  // probabilities of 16 scores (one 32-key block) into two h8
  auto probs16 = [&](const f16x& s, h8* pf, float m_use) {
    float ps0 = 0.f, ps1 = 0.f;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
      for (int j = 0; j < 8; ++j) pf[t][j] = (half_t)__builtin_amdgcn_exp2f(fmaf(s[8 * t + j], c, -m_use));
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
  auto max16 = [&](const f16x& s) {
    float mx = s[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, s[r]);
    return pair_max(mx);
  };
  auto softmax16 = [&](const f16x& s, h8* pf) {
    float psum = probs16(s, pf, m_run);
    if (__builtin_amdgcn_ballot_w64(!(psum <= kLazyLimit)) != 0) {
      const float m_new = fmaxf(m_run, max16(s) * c);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      psum = probs16(s, pf, m_new);
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db] *= alpha;
      l_run *= alpha;
      m_run = m_new;
    }
    l_run += psum;
  };
  auto softmax32 = [&](const f16x (&s)[2], h8 (&pf)[4]) {
    float psum = probs16(s[0], pf, m_run) + probs16(s[1], pf + 2, m_run);
    if (__builtin_amdgcn_ballot_w64(!(psum <= kLazyLimit)) != 0) {
      const float m_new = fmaxf(m_run, fmaxf(max16(s[0]), max16(s[1])) * c);
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      psum = probs16(s[0], pf, m_new) + probs16(s[1], pf + 2, m_new);
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db] *= alpha;
      l_run *= alpha;
      m_run = m_new;
    }
    l_run += psum;
  };

  if constexpr (MODE == 0) {
    f16x sA[2], sB[2];
    h8 pA[4], pB[4];
    qk(sK0, sA);
    auto body = [&](auto bc, f16x (&s_cur)[2], f16x (&s_nxt)[2], h8 (&p_cur)[4], const h8 (&p_prev)[4], bool with_pv) {
      constexpr int B = decltype(bc)::value;
      __syncthreads();
      qk(B == 0 ? sK1 : sK0, s_nxt);
      if (with_pv) pv(B == 0 ? sV1 : sV0, p_prev, 0, 4);
      softmax32(s_cur, p_cur);
    };
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    body(I0{}, sA, sB, pA, pB, false);
    for (int it = 1; it < ntiles; it += 2) {
      body(I1{}, sB, sA, pB, pA, true);
      body(I0{}, sA, sB, pA, pB, true);
    }
  } else if constexpr (MODE == 1) {
    f16x s[2];
    h8 pf[4];
    for (int it = 0; it < ntiles; it += 2) {
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        __syncthreads();
        qk(b == 0 ? sK0 : sK1, s);
        softmax32(s, pf);
        __syncthreads();
        pv(sV0, pf, 0, 4);
      }
    }
  } else {
    f16x s;
    h8 pf[2];
    for (int it = 0; it < ntiles; it += 2) {
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const char* kt = b == 0 ? sK0 : sK1;
        __syncthreads();
        qk_half(kt, s, 0);
        softmax16(s, pf);
        __syncthreads();
        pv(sV0, pf, 0, 2);
        qk_half(kt, s, 1);
        softmax16(s, pf);
        pv(sV0, pf, 2, 4);
      }
    }
  }
  float acc = l_run + m_run;
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc += o[db][r];
  out[blockIdx.x * 256 + tid] = acc;
}

#define CHECK(x)                                                         \
  do {                                                                   \
    hipError_t e_ = (x);                                                 \
    if (e_ != hipSuccess) {                                              \
      fprintf(stderr, "%s: %s\n", #x, hipGetErrorString(e_));           \
      return 1;                                                          \
    }                                                                    \
  } while (0)

int main(int argc, char** argv) {
  if (argc != 4) {
    fprintf(stderr, "usage: %s MODE(0-2) NTILES WORKGROUPS_PER_CU\n", argv[0]);
    return 2;
  }
  const int mode = atoi(argv[1]), ntiles = atoi(argv[2]), per_cu = atoi(argv[3]);
  if (mode < 0 || mode > 2 || ntiles < 1 || ntiles > 100000 || per_cu < 1 || per_cu > (mode == 0 ? 2 : 3)) {
    fprintf(stderr, "MODE 0-2, NTILES 1-100000, WORKGROUPS_PER_CU 1-2 (MODE 0) or 1-3\n");
    return 2;
  }
  hipDeviceProp_t prop;
  CHECK(hipGetDeviceProperties(&prop, 0));
  const int grid = prop.multiProcessorCount * per_cu;
  h8* q;
  float* out;
  CHECK(hipMalloc(&q, (size_t)grid * 256 * 8 * sizeof(h8)));
  CHECK(hipMalloc(&out, (size_t)grid * 256 * sizeof(float)));
  CHECK(hipMemset(q, 0x2A, (size_t)grid * 256 * 8 * sizeof(h8)));  // Q elements 0.0464
  auto launch = [&]() {
    if (mode == 0) hipLaunchKernelGGL(mb<0>, dim3(grid), dim3(256), 0, 0, q, out, ntiles, 0.18f);
    else if (mode == 1) hipLaunchKernelGGL(mb<1>, dim3(grid), dim3(256), 0, 0, q, out, ntiles, 0.18f);
    else hipLaunchKernelGGL(mb<2>, dim3(grid), dim3(256), 0, 0, q, out, ntiles, 0.18f);
  };
  launch();
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  CHECK(hipEventRecord(e0, 0));
  for (int r = 0; r < 5; ++r) launch();
  CHECK(hipEventRecord(e1, 0));
  CHECK(hipEventSynchronize(e1));
  float ms;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  const double us = ms * 1000.0 / 5;
  // flops: per WG per tile 2 heads x 64 rows x 64 keys x 128 x 2 (QK, PV) x 2
  const double flops = (double)grid * ntiles * 4.0 * 32 * 64 * 128 * 2 * 2;
  printf("mode %d tiles %d wgs/cu %d grid %d: %.1f us, %.3f us per tile-step, %.0f TFLOP/s (%.3f of 2.5 PF)\n", mode,
         ntiles, per_cu, grid, us, us / ntiles, flops / us * 1e-6, flops / us * 1e-6 / 2500.0);
  CHECK(hipGetLastError());
  CHECK(hipFree(q));
  CHECK(hipFree(out));
  return 0;
}
