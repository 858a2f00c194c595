// oxs_lm_head.hip — the LM head that feeds the sampler, in the reference CUDA
// backend's GGUF formats (Q8_0 weights x q8_1 activations), on gfx950.
//
// The reference's batched decode quantizes the final hidden states to q8_1
// and projects them with launch_cuda_mmvq_q8_0
// (oxide-backend-cuda/src/lib.rs:4013-4035). Here:
// - quantize_q8_1_kernel: one 32-lane group per q8_1 block, amax and sum by
//   the same xor butterfly, so the stored sum is the reference's bit for bit;
// - pack_q8_0_kernel: a one-time repack of the GGUF rows into tiles of 32
//   tokens x one 32-wide k block, with the quants in the order the matrix
//   cores read them (one 16-byte load per lane per block) and the 32 scales
//   permuted to the rows each lane's accumulators hold;
// - mmvq_q8_0_kernel: per wavefront 32 tokens x 32 batch columns. Each k block
//   is one v_mfma_i32_32x32x32_i8, giving the exact integer dot of every
//   (token, column) pair; the float accumulation then follows the reference
//   kernel exactly (four accumulators by b % 4, fmaf(d_w * d_x, dot, acc),
//   then (A0 + A2) + (A1 + A3)), so y is the reference's to the last bit.
//
// Bound: HBM (34 bytes per 32 weights, read once; activations and y are small
// beside them) and, as the batch grows, the VALU's operations per
// (token, column, block) that the reference's float order needs (convert the
// integer dot, scale product, fused multiply-add).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/oxide_sampler.h"

namespace oxs_lm {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kQ81Bytes = 36;       // {f16 d, f16 sum, int8 qs[32]} (common_types.cuh:8-11)
constexpr int kQ80Bytes = 34;       // {f16 d, int8 qs[32]} (common_types.cuh:13-16)
constexpr int kPackedBlock = 1088;  // 32 tokens x one k block: 64 lanes x 16 quant bytes, then 32 f16 scales
constexpr int kGroupsPerBlock = 4;  // token groups (wavefronts) per workgroup
constexpr int kThreads = 256;

__device__ __forceinline__ float half_to_float(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// (float)half(lo or hi 16 bits of w) * x, rounded once, in one v_fma_mix_f32
// (S0 read as f16, S1 as f32, S2 = 0): the widening is exact, so this equals
// the multiply after a conversion, except that a zero product is +0; the
// accumulators start at +0 and a +0 or -0 product leaves them equal.
template <int HI>
__device__ __forceinline__ float half_times(uint32_t w, float x) {
  float d;
  if constexpr (HI)
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(d) : "v"(w), "v"(x));
  else
    asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[1,0,0]" : "=v"(d) : "v"(w), "v"(x));
  return d;
}
__device__ __forceinline__ uint16_t float_to_half(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// Row i of the 32 x 32 MFMA output held in register r of a lane in half g
// (lanes 32g .. 32g + 31): 8 (r / 4) + 4 g + r % 4.
__device__ __forceinline__ uint32_t out_row(uint32_t r, uint32_t g) { return 8u * (r >> 2) + 4u * g + (r & 3u); }

// quantize_f32_to_q8_1_cuda_kernel (norms_rope.cu:2-29): eight 32-lane groups
// per workgroup, one q8_1 block each.
__global__ __launch_bounds__(kThreads) void quantize_q8_1_kernel(const float* __restrict__ x, uint32_t nblocks,
                                                                 uint8_t* __restrict__ y) {
  const uint32_t lane = threadIdx.x & 31u;
  const uint32_t blk = blockIdx.x * (kThreads / 32) + (threadIdx.x >> 5);
  if (blk >= nblocks) return;  // the whole 32-lane group leaves together
  const float v = x[(size_t)blk * 32 + lane];
  float amax = fabsf(v), sum = v;
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) {
    amax = fmaxf(amax, __shfl_xor(amax, o, 32));
    sum += __shfl_xor(sum, o, 32);
  }
  const float d = amax / 127.0f;
  const float id = d > 0.0f ? 1.0f / d : 0.0f;
  uint8_t* out = y + (size_t)blk * kQ81Bytes;
  out[4 + lane] = (uint8_t)(int8_t)roundf(v * id);
  if (lane == 0) {
    *(uint16_t*)out = float_to_half(d);
    *(uint16_t*)(out + 2) = float_to_half(sum);
  }
}

// One wavefront per (token group, k block): lane l writes quant bytes
// [16 (l / 32), +16) of token 32 tg + l % 32 at offset 16 l; lanes 0..31 write
// the scales, position p holding token out_row(p % 16, p / 16). Tokens past m
// are zero.
__global__ __launch_bounds__(kThreads) void pack_q8_0_kernel(const uint8_t* __restrict__ w, uint32_t m, uint32_t nb,
                                                             uint64_t pieces, uint8_t* __restrict__ out) {
  const uint64_t gid = (uint64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
  if (gid >= pieces) return;
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t tg = (uint32_t)(gid / nb), b = (uint32_t)(gid % nb);
  uint8_t* dst = out + gid * kPackedBlock;
  {
    const uint32_t t = tg * 32u + (lane & 31u), g = lane >> 5;
    uint32_t q[4] = {0u, 0u, 0u, 0u};
    if (t < m) {
      const uint8_t* src = w + ((size_t)t * nb + b) * kQ80Bytes + 2 + 16 * g;  // 2-byte aligned
#pragma unroll
      for (int i = 0; i < 16; ++i) q[i / 4] |= (uint32_t)src[i] << (8 * (i % 4));
    }
    *(uint4*)(dst + 16 * lane) = make_uint4(q[0], q[1], q[2], q[3]);
  }
  if (lane < 32) {
    const uint32_t t = tg * 32u + out_row(lane & 15u, lane >> 4);
    uint16_t s = 0;
    if (t < m) {
      const uint8_t* src = w + ((size_t)t * nb + b) * kQ80Bytes;
      s = (uint16_t)(src[0] | (src[1] << 8));
    }
    *(uint16_t*)(dst + 1024 + 2 * lane) = s;
  }
}

// mmvq_q8_0_cuda_kernel (quant_gemv_standard.cu:425-513) for 32 columns x
// 128 tokens per workgroup; each wavefront owns one group of 32 tokens. With
// a batch above 32 columns, the workgroups of one token range sit 8 apart in
// launch order: workgroups go round-robin over the 8 XCDs, so they run on
// the same XCD at about the same time and the second reads the weights from
// that XCD's L2 instead of HBM.
// - The activations of a group of four k blocks are staged once per
//   workgroup in LDS (double-buffered, one barrier per group): quants as
//   [k block][half g][column][16 bytes], scales converted to float.
// - Each wavefront loads the next group's weights (one 16-byte load per lane
//   per block, plus 32 bytes of scales) while it computes the current one.
// Wavefronts past the last token group skip the arithmetic and stores but
// keep taking part in the staging and the barriers.
constexpr int kGroupBlocks = 4;  // k blocks per pipeline step (one per accumulator)

__global__ __launch_bounds__(kThreads) void mmvq_q8_0_kernel(float* __restrict__ y, const uint8_t* __restrict__ wp,
                                                             const uint8_t* __restrict__ x, uint32_t m, uint32_t nb,
                                                             uint32_t batch, uint32_t ncb, uint32_t vec_out) {
  constexpr int TILES = 1;
  constexpr int COLS = 32 * TILES;
  __shared__ __align__(16) uint4 s_xq[2][kGroupBlocks][2][COLS];  // quant halves
  __shared__ float s_xd[2][kGroupBlocks][COLS];                   // scales as float
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  // token block tb and column block cb: in each run of 8 * ncb workgroups,
  // workgroup 8 c + i holds token block i of the run and column block c
  uint32_t tb, cb;
  {
    const uint32_t per = 8u * ncb, full = (gridDim.x / per) * per;
    if (blockIdx.x < full) {
      const uint32_t run = blockIdx.x / per, r = blockIdx.x - run * per;
      tb = run * 8u + (r & 7u);
      cb = r >> 3;
    } else {
      const uint32_t r = blockIdx.x - full;
      tb = (full / per) * 8u + r / ncb;
      cb = r - (r / ncb) * ncb;
    }
  }
  const uint32_t tg = tb * kGroupsPerBlock + wave;
  const bool live = tg < (m + 31u) / 32u;
  const uint32_t g = lane >> 5, j = lane & 31u;
  const uint32_t c0 = cb * COLS;
  const uint32_t ngroups = nb / kGroupBlocks;

  // staging: thread t < COLS * 4 copies the q8_1 block (column t / 4, block t % 4) of each group
  const bool stager = tid < (uint32_t)(COLS * kGroupBlocks);
  const uint32_t st_col = tid / kGroupBlocks, st_kb = tid % kGroupBlocks;
  const uint8_t* st_src = x + (size_t)min(c0 + st_col, batch - 1u) * nb * kQ81Bytes + (size_t)st_kb * kQ81Bytes;
  uint32_t xr[9];
  auto stage_load = [&](uint32_t grp) {
    if (stager) {
      const uint32_t* p = (const uint32_t*)(st_src + (size_t)grp * kGroupBlocks * kQ81Bytes);  // 4-byte aligned
#pragma unroll
      for (int i = 0; i < 9; ++i) xr[i] = p[i];
    }
  };
  auto stage_store = [&](int buf) {
    if (stager) {
      s_xd[buf][st_kb][st_col] = half_to_float((uint16_t)(xr[0] & 0xffffu));
      s_xq[buf][st_kb][0][st_col] = make_uint4(xr[1], xr[2], xr[3], xr[4]);
      s_xq[buf][st_kb][1][st_col] = make_uint4(xr[5], xr[6], xr[7], xr[8]);
    }
  };

  const uint8_t* wg = wp + (size_t)(live ? tg : 0u) * nb * kPackedBlock;
  v4i wa[kGroupBlocks];
  uint4 ws0[kGroupBlocks], ws1[kGroupBlocks];
  auto weight_load = [&](uint32_t grp) {
#pragma unroll
    for (int q = 0; q < kGroupBlocks; ++q) {
      const uint8_t* blk = wg + (size_t)(grp * kGroupBlocks + q) * kPackedBlock;
      wa[q] = *(const v4i*)(blk + 16 * lane);
      ws0[q] = *(const uint4*)(blk + 1024 + 32 * g);
      ws1[q] = *(const uint4*)(blk + 1024 + 32 * g + 16);
    }
  };

  float acc[TILES][kGroupBlocks][16];
#pragma unroll
  for (int t = 0; t < TILES; ++t)
#pragma unroll
    for (int q = 0; q < kGroupBlocks; ++q)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[t][q][r] = 0.0f;
  const v16i zero = {};

  stage_load(0);
  stage_store(0);
  if (live) weight_load(0);
  __syncthreads();
  for (uint32_t grp = 0; grp < ngroups; ++grp) {
    const int buf = grp & 1;
    v4i ca[kGroupBlocks];
    uint4 cs0[kGroupBlocks], cs1[kGroupBlocks];
#pragma unroll
    for (int q = 0; q < kGroupBlocks; ++q) {
      ca[q] = wa[q];
      cs0[q] = ws0[q];
      cs1[q] = ws1[q];
    }
    const bool more = grp + 1 < ngroups;
    if (more) {
      stage_load(grp + 1);
      if (live) weight_load(grp + 1);
    }
    if (live) {
#pragma unroll
      for (int q = 0; q < kGroupBlocks; ++q) {
        const uint32_t sw[8] = {cs0[q].x, cs0[q].y, cs0[q].z, cs0[q].w, cs1[q].x, cs1[q].y, cs1[q].z, cs1[q].w};
#pragma unroll
        for (int t = 0; t < TILES; ++t) {
          const uint4 bq = s_xq[buf][q][g][32 * t + j];
          const float dx = s_xd[buf][q][32 * t + j];
          const v4i bv = {(int)bq.x, (int)bq.y, (int)bq.z, (int)bq.w};
          const v16i d = __builtin_amdgcn_mfma_i32_32x32x32_i8(ca[q], bv, zero, 0, 0, 0);
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float dd = (r % 2) ? half_times<1>(sw[r / 2], dx) : half_times<0>(sw[r / 2], dx);
            acc[t][q][r] = __builtin_fmaf(dd, (float)d[r], acc[t][q][r]);
          }
        }
      }
    }
    if (more) stage_store(buf ^ 1);
    __syncthreads();
  }
  if (!live) return;

  // (A0 + A2) + (A1 + A3); registers 4 q' .. 4 q' + 3 hold four consecutive tokens
  const bool vec = vec_out != 0u;  // m % 4 == 0 and y 16-byte aligned: float4 stores
#pragma unroll
  for (int t = 0; t < TILES; ++t) {
    const uint32_t col = c0 + 32u * t + j;
    if (col >= batch) continue;
    float* yrow = y + (size_t)col * m;
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = 4 * qq + e;
        v[e] = (acc[t][0][r] + acc[t][2][r]) + (acc[t][1][r] + acc[t][3][r]);
      }
      const uint32_t tok = tg * 32u + out_row(4u * qq, g);
      if (vec && tok + 3u < m) {
        *(float4*)(yrow + tok) = make_float4(v[0], v[1], v[2], v[3]);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (tok + e < m) yrow[tok + e] = v[e];
      }
    }
  }
}

// The same product for batches of at most four columns, where a 32-column
// MFMA tile would be mostly idle (eight columns was measured slower than the
// MFMA kernel). Each workgroup first stages the whole of x
// (NC columns x every k block) in LDS, then each wavefront walks its 32
// tokens with no further barrier: lane (j, g) takes 16 quant bytes of token j
// per block (the packed layout's MFMA order), four dot4 products per column,
// and the lane pair (j, j + 32) adds its halves into the block's exact
// integer dot. The float accumulation is the reference's, as above. Bound:
// HBM.
template <int NC>
__global__ __launch_bounds__(kThreads) void mmvq_q8_0_small_kernel(float* __restrict__ y,
                                                                   const uint8_t* __restrict__ wp,
                                                                   const uint8_t* __restrict__ x, uint32_t m,
                                                                   uint32_t nb, uint32_t batch) {
  extern __shared__ __align__(16) uint8_t s_small[];
  uint4* s_q = (uint4*)s_small;                              // [NC][nb][2] quant halves
  float* s_d = (float*)(s_small + (size_t)NC * nb * 32);     // [NC][nb] scales
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  for (uint32_t i = tid; i < NC * nb; i += kThreads) {
    const uint32_t c = i / nb, b = i - c * nb;
    const uint32_t* p = (const uint32_t*)(x + ((size_t)min(c, batch - 1u) * nb + b) * kQ81Bytes);
    s_d[i] = half_to_float((uint16_t)(p[0] & 0xffffu));
    s_q[2 * i] = make_uint4(p[1], p[2], p[3], p[4]);
    s_q[2 * i + 1] = make_uint4(p[5], p[6], p[7], p[8]);
  }
  __syncthreads();
  const uint32_t tg = blockIdx.x * kGroupsPerBlock + wave;
  if (tg >= (m + 31u) / 32u) return;
  const uint32_t g = lane >> 5, j = lane & 31u;
  // this token's scale: position 16 ((j / 4) % 2) + 4 (j / 8) + j % 4 of the permuted scales
  const uint32_t sp = 16u * ((j >> 2) & 1u) + 4u * (j >> 3) + (j & 3u);
  const uint8_t* wg = wp + (size_t)tg * nb * kPackedBlock;
  float acc[NC][4];
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int q = 0; q < 4; ++q) acc[c][q] = 0.0f;
  for (uint32_t b0 = 0; b0 < nb; b0 += 4) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t b = b0 + q;
      const uint8_t* blk = wg + (size_t)b * kPackedBlock;
      const uint4 wq = *(const uint4*)(blk + 16 * lane);
      const float dw = half_to_float(*(const uint16_t*)(blk + 1024 + 2 * sp));
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const uint4 xq = s_q[2 * (c * nb + b) + g];
        int dot = __builtin_amdgcn_sdot4((int)wq.x, (int)xq.x, 0, false);
        dot = __builtin_amdgcn_sdot4((int)wq.y, (int)xq.y, dot, false);
        dot = __builtin_amdgcn_sdot4((int)wq.z, (int)xq.z, dot, false);
        dot = __builtin_amdgcn_sdot4((int)wq.w, (int)xq.w, dot, false);
        dot += __shfl_xor(dot, 32);
        acc[c][q] = __builtin_fmaf(dw * s_d[c * nb + b], (float)dot, acc[c][q]);
      }
    }
  }
  const uint32_t tok = tg * 32u + j;
  if (g == 0 && tok < m) {
#pragma unroll
    for (int c = 0; c < NC; ++c)
      if ((uint32_t)c < batch) y[(size_t)c * m + tok] = (acc[c][0] + acc[c][2]) + (acc[c][1] + acc[c][3]);
  }
}

}  // namespace oxs_lm

static int launch_status() { return hipGetLastError() == hipSuccess ? OXS_OK : OXS_ERR_HIP; }

extern "C" int oxs_quantize_q8_1(const float* x, uint32_t n, void* y_q8_1, void* stream) {
  const uint32_t nblocks = n / 32u;
  if (nblocks == 0) return OXS_OK;
  if (!x || !y_q8_1) return OXS_ERR_INVALID_ARGUMENT;
  if (((uintptr_t)x & 3u) || ((uintptr_t)y_q8_1 & 1u)) return OXS_ERR_INVALID_ARGUMENT;  // float loads, half stores
  const uint32_t per = oxs_lm::kThreads / 32;
  hipLaunchKernelGGL(oxs_lm::quantize_q8_1_kernel, dim3((nblocks + per - 1) / per), dim3(oxs_lm::kThreads), 0,
                     (hipStream_t)stream, x, nblocks, (uint8_t*)y_q8_1);
  return launch_status();
}

extern "C" size_t oxs_q8_0_packed_bytes(uint32_t m, uint32_t k) {
  if (k == 0 || k % 128u != 0) return 0;
  return (size_t)((m + 31u) / 32u) * (k / 32u) * oxs_lm::kPackedBlock;
}

extern "C" int oxs_pack_q8_0(const void* w, uint32_t m, uint32_t k, void* w_packed, void* stream) {
  if (k == 0 || k % 128u != 0) return OXS_ERR_UNSUPPORTED;
  if (m == 0) return OXS_OK;
  if (!w || !w_packed) return OXS_ERR_INVALID_ARGUMENT;
  if ((uintptr_t)w_packed & 15u) return OXS_ERR_INVALID_ARGUMENT;  // 16-byte stores
  const uint32_t nb = k / 32u;
  const uint64_t pieces = (uint64_t)((m + 31u) / 32u) * nb;
  const uint64_t per = oxs_lm::kThreads / 64;
  const uint64_t grid = (pieces + per - 1) / per;
  if (grid > 0x7fffffffull) return OXS_ERR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(oxs_lm::pack_q8_0_kernel, dim3((uint32_t)grid), dim3(oxs_lm::kThreads), 0, (hipStream_t)stream,
                     (const uint8_t*)w, m, nb, pieces, (uint8_t*)w_packed);
  return launch_status();
}

extern "C" int oxs_mmvq_q8_0(float* y, const void* w_packed, const void* x_q8_1, uint32_t m, uint32_t k,
                             uint32_t batch, void* stream) {
  if (m == 0 || k == 0 || batch == 0) return OXS_OK;  // as launch_cuda_mmvq_q8_0's early return
  if (k % 128u != 0) return OXS_ERR_UNSUPPORTED;
  if (!y || !w_packed || !x_q8_1) return OXS_ERR_INVALID_ARGUMENT;
  // 16-byte weight loads, 4-byte activation loads, 4-byte stores
  if (((uintptr_t)w_packed & 15u) || ((uintptr_t)x_q8_1 & 3u) || ((uintptr_t)y & 3u)) return OXS_ERR_INVALID_ARGUMENT;
  const uint32_t vec_out = (m % 4u == 0u && ((uintptr_t)y & 15u) == 0u) ? 1u : 0u;
  const uint32_t groups = (m + 31u) / 32u;
  const uint32_t gx = (groups + oxs_lm::kGroupsPerBlock - 1) / oxs_lm::kGroupsPerBlock;
  const uint32_t nc_small = batch <= 1u ? 1u : batch <= 2u ? 2u : 4u;  // columns the small kernel stages
  if (batch <= 4u && (size_t)nc_small * (k / 32u) * 36u <= 65536u) {    // the whole of x fits in LDS
    const uint32_t nb = k / 32u;
    const size_t lds = (size_t)nc_small * nb * 36u;
    const dim3 g1(gx);
    switch (batch) {
      case 1: hipLaunchKernelGGL(oxs_lm::mmvq_q8_0_small_kernel<1>, g1, dim3(oxs_lm::kThreads), lds,
                                 (hipStream_t)stream, y, (const uint8_t*)w_packed, (const uint8_t*)x_q8_1, m, nb,
                                 batch); break;
      case 2: hipLaunchKernelGGL(oxs_lm::mmvq_q8_0_small_kernel<2>, g1, dim3(oxs_lm::kThreads), lds,
                                 (hipStream_t)stream, y, (const uint8_t*)w_packed, (const uint8_t*)x_q8_1, m, nb,
                                 batch); break;
      default: hipLaunchKernelGGL(oxs_lm::mmvq_q8_0_small_kernel<4>, g1, dim3(oxs_lm::kThreads), lds,
                                  (hipStream_t)stream, y, (const uint8_t*)w_packed, (const uint8_t*)x_q8_1, m, nb,
                                  batch); break;
    }
    return launch_status();
  }
  const uint32_t ncb = (batch + 31u) / 32u;  // 32-column blocks
  const uint64_t grid = (uint64_t)gx * ncb;
  if (grid > 0x7fffffffull) return OXS_ERR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(oxs_lm::mmvq_q8_0_kernel, dim3((uint32_t)grid), dim3(oxs_lm::kThreads), 0, (hipStream_t)stream,
                     y, (const uint8_t*)w_packed, (const uint8_t*)x_q8_1, m, k / 32u, batch, ncb, vec_out);
  return launch_status();
}
