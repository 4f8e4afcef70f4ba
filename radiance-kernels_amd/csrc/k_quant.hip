// MX quantizers (rules R1 and R4), the KV-cache append and the synthetic-input
// generator.
#pragma once

#include "kernel_base.h"

// ============================================================================
// Quantizers (rule R1).  One MX block of 32 values is handled by 8 lanes.
// ============================================================================
// E4M3 codes of four values x 2^sh, or (FMT 1) E3M2 codes through the table e3m2_tab.
template <int FMT>
__device__ __forceinline__ uint32_t encode4(float4 v, int sh, const uint8_t* e3m2_tab = nullptr) {
  float y[4] = {__builtin_ldexpf(v.x, sh), __builtin_ldexpf(v.y, sh), __builtin_ldexpf(v.z, sh),
                __builtin_ldexpf(v.w, sh)};
  if (FMT == 0) return e4m3_code4(y[0], y[1], y[2], y[3]);
  uint32_t w = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) w |= e3m2_code_tab(y[i], e3m2_tab) << (8 * i);
  return w;
}

// x: rows of `cols` floats, 32-blocks along the row. nblocks = rows * cols / 32.
template <int FMT>
__device__ void quant_rows_impl(const float* __restrict__ x, int64_t nblocks, uint8_t* __restrict__ codes,
                                uint8_t* __restrict__ scales) {
  __shared__ uint8_t e3m2_tab[FMT == 0 ? 4 : E3M2_TAB_N];
  if constexpr (FMT != 0) {
    e3m2_tab_fill(e3m2_tab, threadIdx.x, blockDim.x);
    __syncthreads();
  }
  int64_t gt = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int64_t blk = gt >> 3;
  int part = (int)(gt & 7);
  if (blk >= nblocks) return;                       // whole 8-lane groups leave together
  float4 v = reinterpret_cast<const float4*>(x)[blk * 8 + part];
  float a = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  a = fmaxf(a, __shfl_xor(a, 1));
  a = fmaxf(a, __shfl_xor(a, 2));
  a = fmaxf(a, __shfl_xor(a, 4));
  uint32_t sc = scale_code(a, FMT == 0 ? 8 : 4);
  reinterpret_cast<uint32_t*>(codes)[blk * 8 + part] = encode4<FMT>(v, 127 - (int)sc, e3m2_tab);
  if (part == 0) scales[blk] = (uint8_t)sc;
}

extern "C" __global__ void __launch_bounds__(256) mxfa_quant_rows_e4m3(const float* x, int64_t nblocks,
                                                                       uint8_t* codes, uint8_t* scales) {
  quant_rows_impl<0>(x, nblocks, codes, scales);
}
extern "C" __global__ void __launch_bounds__(256) mxfa_quant_rows_e3m2(const float* x, int64_t nblocks,
                                                                       uint8_t* codes, uint8_t* scales) {
  quant_rows_impl<1>(x, nblocks, codes, scales);
}

// Rule R4 (the reference's SIMT block quantizer), 32-blocks along each row; amax is the
// reference's running "if (|x| > amax)" maximum, which skips NaN like fmaxf.
extern "C" __global__ void __launch_bounds__(256) mxfa_quant_rows_r4(const float* x, int64_t nblocks, uint8_t* codes,
                                                                     uint8_t* scales) {
  const int64_t gt = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t blk = gt >> 3;
  const int part = (int)(gt & 7);
  if (blk >= nblocks) return;                       // whole 8-lane groups leave together
  const float4 v = reinterpret_cast<const float4*>(x)[blk * 8 + part];
  float a = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  a = fmaxf(a, __shfl_xor(a, 1));
  a = fmaxf(a, __shfl_xor(a, 2));
  a = fmaxf(a, __shfl_xor(a, 4));
  float mul;
  const uint32_t sc = r4_scale(a, mul);
  reinterpret_cast<uint32_t*>(codes)[blk * 8 + part] = r4_e4m3_code(v.x * mul) | (r4_e4m3_code(v.y * mul) << 8) |
                                                       (r4_e4m3_code(v.z * mul) << 16) |
                                                       (r4_e4m3_code(v.w * mul) << 24);
  if (part == 0) scales[blk] = (uint8_t)sc;
}

// 32-blocks along rows (V layout).  One wave per (matrix, 32-row block, 128 columns): lane
// (cg, h) = (lane % 32, lane / 32) owns columns 4 cg .. 4 cg + 3 of the group and the 16 rows
// 8 g + 4 h + b (g, b < 4), read once into registers (a load instruction covers 512 contiguous
// bytes of each of two rows); the two row halves combine their amax with one lane swap.
// mats matrices of rows x cols; rows % 32 == 0, cols % 4 == 0 (columns past cols are skipped).
// FMT 2: E3M2, each 32-row block of a column stored as 24 bytes at codes + ((m * rows / 32 +
// rb) * cols + c) * 24, row r's code in field blk6_field(r) (bits 6f .. 6f + 5, little
// endian): the fp6 A operand of the scaled MFMA in the key order of the P operand the
// attention kernels build.  Lane half h's rows are fields 16 h .. 16 h + 15 in row order, i.e.
// 12 contiguous bytes of each of its columns' blocks.
template <int FMT>
__device__ void quant_cols_impl(const float* __restrict__ x, int64_t mats, int rows, int cols,
                                uint8_t* __restrict__ codes, uint8_t* __restrict__ scales) {
  __shared__ uint8_t e3m2_tab[FMT == 0 ? 4 : E3M2_TAB_N];
  if constexpr (FMT != 0) {
    e3m2_tab_fill(e3m2_tab, threadIdx.x, blockDim.x);
    __syncthreads();
  }
  const int lane = threadIdx.x & 63;
  const int64_t unit = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int ncg = (cols + 127) / 128, nrb = rows / 32;
  if (unit >= mats * nrb * ncg) return;                          // whole waves leave together
  const int64_t m = unit / ((int64_t)nrb * ncg);
  const int rem = (int)(unit % ((int64_t)nrb * ncg));
  const int rb = rem / ncg, c4 = (rem % ncg) * 128 + 4 * (lane & 31), h = lane >> 5;
  const bool cok = c4 < cols;
  const float* base = x + (m * rows + (int64_t)rb * 32) * cols + c4;
  float4 v[16];
  float4 amax = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int j = 0; j < 16; j++) {
    const int r = 8 * (j >> 2) + 4 * h + (j & 3);
    v[j] = cok ? *reinterpret_cast<const float4*>(base + (int64_t)r * cols) : make_float4(0.f, 0.f, 0.f, 0.f);
    amax.x = fmaxf(amax.x, fabsf(v[j].x)); amax.y = fmaxf(amax.y, fabsf(v[j].y));
    amax.z = fmaxf(amax.z, fabsf(v[j].z)); amax.w = fmaxf(amax.w, fabsf(v[j].w));
  }
  amax.x = fmaxf(amax.x, __shfl_xor(amax.x, 32)); amax.y = fmaxf(amax.y, __shfl_xor(amax.y, 32));
  amax.z = fmaxf(amax.z, __shfl_xor(amax.z, 32)); amax.w = fmaxf(amax.w, __shfl_xor(amax.w, 32));
  if (!cok) return;
  const int lp = FMT == 0 ? 8 : 4;
  const uint32_t s0 = scale_code(amax.x, lp), s1 = scale_code(amax.y, lp), s2 = scale_code(amax.z, lp),
                 s3 = scale_code(amax.w, lp);
  if (h == 0)
    *reinterpret_cast<uint32_t*>(scales + (m * nrb + rb) * cols + c4) = s0 | (s1 << 8) | (s2 << 16) | (s3 << 24);
  if constexpr (FMT == 2) {
    uint32_t pk[4][3] = {};
#pragma unroll
    for (int j = 0; j < 16; j++) {
      const uint32_t c[4] = {e3m2_code_tab(__builtin_ldexpf(v[j].x, 127 - (int)s0), e3m2_tab),
                             e3m2_code_tab(__builtin_ldexpf(v[j].y, 127 - (int)s1), e3m2_tab),
                             e3m2_code_tab(__builtin_ldexpf(v[j].z, 127 - (int)s2), e3m2_tab),
                             e3m2_code_tab(__builtin_ldexpf(v[j].w, 127 - (int)s3), e3m2_tab)};
      // local field j: bits 6 j of the lane's 96
      const int bit = 6 * j;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        pk[q][bit / 32] |= c[q] << (bit % 32);
        if (bit % 32 > 26) pk[q][bit / 32 + 1] |= c[q] >> (32 - bit % 32);
      }
    }
#pragma unroll
    for (int q = 0; q < 4; q++) {
      uint32_t* dst = reinterpret_cast<uint32_t*>(codes + ((m * nrb + rb) * cols + c4 + q) * 24 + 12 * h);
      dst[0] = pk[q][0];
      dst[1] = pk[q][1];
      dst[2] = pk[q][2];
    }
    return;
  }
  uint8_t* cbase = codes + (m * rows + (int64_t)rb * 32) * cols + c4;
#pragma unroll
  for (int j = 0; j < 16; j++) {
    const int r = 8 * (j >> 2) + 4 * h + (j & 3);
    const float y0 = __builtin_ldexpf(v[j].x, 127 - (int)s0), y1 = __builtin_ldexpf(v[j].y, 127 - (int)s1);
    const float y2 = __builtin_ldexpf(v[j].z, 127 - (int)s2), y3 = __builtin_ldexpf(v[j].w, 127 - (int)s3);
    uint32_t w;
    if constexpr (FMT == 0)
      w = e4m3_code4(y0, y1, y2, y3);
    else
      w = e3m2_code_tab(y0, e3m2_tab) | (e3m2_code_tab(y1, e3m2_tab) << 8) | (e3m2_code_tab(y2, e3m2_tab) << 16) |
          (e3m2_code_tab(y3, e3m2_tab) << 24);
    *reinterpret_cast<uint32_t*>(cbase + (int64_t)r * cols) = w;
  }
}

extern "C" __global__ void __launch_bounds__(256) mxfa_quant_cols_e4m3(const float* x, int64_t mats, int rows, int cols,
                                                                       uint8_t* codes, uint8_t* scales) {
  quant_cols_impl<0>(x, mats, rows, cols, codes, scales);
}
extern "C" __global__ void __launch_bounds__(256) mxfa_quant_cols_e3m2(const float* x, int64_t mats, int rows, int cols,
                                                                       uint8_t* codes, uint8_t* scales) {
  quant_cols_impl<1>(x, mats, rows, cols, codes, scales);
}
extern "C" __global__ void __launch_bounds__(256) mxfa_quant_cols_e3m2_blk(const float* x, int64_t mats, int rows,
                                                                           int cols, uint8_t* codes, uint8_t* scales) {
  quant_cols_impl<2>(x, mats, rows, cols, codes, scales);
}

// ============================================================================
// KV-cache append (rule R1).  K: each new token's row is quantized into cache row
// pos0 + i (32-blocks along D).  V: every 32-token block touched by the append is
// re-quantized as a whole from the open block's fp32 tail (positions before pos0), the new
// tokens, and zeros for positions not appended yet (zeros leave R1's amax unchanged), so
// the cache always equals the R1 quantization of the sequence so far.  The block left
// open keeps its fp32 values in the tail: written by the same threads when the append
// touches one block (each lane rewrites only the tail rows and columns it read), by a
// second, stream-ordered kernel when it spans several (the old tail rows are read by the
// first block's threads, the new ones belong to the last block).
// One launch: workgroups [0, kgroups) do K, the rest V.
// ============================================================================
__device__ __forceinline__ void kv_append_k_part(const float* k_new, int64_t gt, int64_t nblocks, int n_new, int L,
                                                 int D, int pos0, uint8_t* k_cache, uint8_t* k_sc) {
  const int64_t blk = gt >> 3;
  const int part = (int)(gt & 7);
  if (blk >= nblocks) return;                       // whole 8-lane groups leave together
  const int bpr = D / 32;
  const int64_t row = blk / bpr;                    // (b * Hkv + kvh) * n_new + i
  const int cb = (int)(blk % bpr);
  const int64_t bk = row / n_new;
  const int i = (int)(row % n_new);
  const float4 v = reinterpret_cast<const float4*>(k_new + row * D + cb * 32)[part];
  float a = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  a = fmaxf(a, __shfl_xor(a, 1));
  a = fmaxf(a, __shfl_xor(a, 2));
  a = fmaxf(a, __shfl_xor(a, 4));
  const uint32_t sc = scale_code(a, 8);
  const int64_t crow = bk * L + pos0 + i;
  reinterpret_cast<uint32_t*>(k_cache + crow * D + cb * 32)[part] = encode4<0>(v, 127 - (int)sc);
  if (part == 0) k_sc[crow * bpr + cb] = (uint8_t)sc;
}

// V: 64-lane units, each = 8 column groups of 4 x 8 row lanes of 4 rows of one (b * Hkv + kvh,
// touched block); lane = cgl + 8 * rl.  Units per (bk, block) = D / 32.
template <int FMT>
__device__ __forceinline__ void kv_append_v_part(const float* v_new, float* v_tail, int64_t unit, int64_t nunits,
                                                 int lane, int ntouch, int n_new, int L, int D, int pos0,
                                                 uint8_t* v_cache, uint8_t* v_sc, const uint8_t* e3m2_tab) {
  if (unit >= nunits) return;                       // whole waves leave together
  const int upb = D / 32;
  const int64_t bk = unit / ((int64_t)ntouch * upb);
  const int rem = (int)(unit % ((int64_t)ntouch * upb));
  const int jb = rem / upb;
  const int cgl = lane & 7, rl = lane >> 3;
  const int c4 = (rem % upb) * 32 + cgl * 4;
  const int end = pos0 + n_new;
  const int blk = pos0 / 32 + jb;
  const int p0 = blk * 32;
  const int tail0 = (pos0 / 32) * 32;               // first position held by the tail
  float4 x[4];
  float4 amax = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int p = p0 + 4 * rl + i;
    if (p < pos0)
      x[i] = *reinterpret_cast<const float4*>(v_tail + (bk * 32 + (p - tail0)) * D + c4);
    else if (p < end)
      x[i] = *reinterpret_cast<const float4*>(v_new + (bk * n_new + (p - pos0)) * D + c4);
    else
      x[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    amax.x = fmaxf(amax.x, fabsf(x[i].x)); amax.y = fmaxf(amax.y, fabsf(x[i].y));
    amax.z = fmaxf(amax.z, fabsf(x[i].z)); amax.w = fmaxf(amax.w, fabsf(x[i].w));
  }
#pragma unroll
  for (int m = 8; m < 64; m <<= 1) {
    amax.x = fmaxf(amax.x, __shfl_xor(amax.x, m)); amax.y = fmaxf(amax.y, __shfl_xor(amax.y, m));
    amax.z = fmaxf(amax.z, __shfl_xor(amax.z, m)); amax.w = fmaxf(amax.w, __shfl_xor(amax.w, m));
  }
  const int lp = FMT == 0 ? 8 : 4;
  const uint32_t s0 = scale_code(amax.x, lp), s1 = scale_code(amax.y, lp), s2 = scale_code(amax.z, lp),
                 s3 = scale_code(amax.w, lp);
  const bool tail_here = ntouch == 1 && (end % 32) != 0;
  if constexpr (FMT == 2) {
    // rows 4 rl .. 4 rl + 3 of a column are the consecutive fields blk6_field(4 rl) .. + 3 of
    // its 24-byte block: three bytes per column at byte 12 (rl % 2) + 3 (rl / 2)
    uint32_t pk[4] = {0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t c[4] = {e3m2_code_tab(__builtin_ldexpf(x[i].x, 127 - (int)s0), e3m2_tab),
                             e3m2_code_tab(__builtin_ldexpf(x[i].y, 127 - (int)s1), e3m2_tab),
                             e3m2_code_tab(__builtin_ldexpf(x[i].z, 127 - (int)s2), e3m2_tab),
                             e3m2_code_tab(__builtin_ldexpf(x[i].w, 127 - (int)s3), e3m2_tab)};
#pragma unroll
      for (int q = 0; q < 4; q++) pk[q] |= c[q] << (6 * i);
      if (tail_here && p0 + 4 * rl + i >= pos0) *reinterpret_cast<float4*>(v_tail + (bk * 32 + 4 * rl + i) * D + c4) = x[i];
    }
#pragma unroll
    for (int q = 0; q < 4; q++) {
      uint8_t* dst = v_cache + ((bk * (L / 32) + blk) * D + c4 + q) * 24 + 12 * (rl & 1) + 3 * (rl >> 1);
      dst[0] = (uint8_t)pk[q];
      dst[1] = (uint8_t)(pk[q] >> 8);
      dst[2] = (uint8_t)(pk[q] >> 16);
    }
    if (rl == 0)
      *reinterpret_cast<uint32_t*>(v_sc + (bk * (L / 32) + blk) * D + c4) = s0 | (s1 << 8) | (s2 << 16) | (s3 << 24);
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = 4 * rl + i;
    const float y0 = __builtin_ldexpf(x[i].x, 127 - (int)s0), y1 = __builtin_ldexpf(x[i].y, 127 - (int)s1);
    const float y2 = __builtin_ldexpf(x[i].z, 127 - (int)s2), y3 = __builtin_ldexpf(x[i].w, 127 - (int)s3);
    uint32_t w;
    if constexpr (FMT == 0)
      w = e4m3_code4(y0, y1, y2, y3);
    else
      w = e3m2_code_tab(y0, e3m2_tab) | (e3m2_code_tab(y1, e3m2_tab) << 8) | (e3m2_code_tab(y2, e3m2_tab) << 16) |
          (e3m2_code_tab(y3, e3m2_tab) << 24);
    *reinterpret_cast<uint32_t*>(v_cache + (bk * L + p0 + r) * D + c4) = w;
    if (tail_here && p0 + r >= pos0) *reinterpret_cast<float4*>(v_tail + (bk * 32 + r) * D + c4) = x[i];
  }
  if (rl == 0)
    *reinterpret_cast<uint32_t*>(v_sc + (bk * (L / 32) + blk) * D + c4) = s0 | (s1 << 8) | (s2 << 16) | (s3 << 24);
}

template <int FMT>
__device__ void kv_append_impl(const float* k_new, const float* v_new, float* v_tail, int64_t kblocks, int kgroups,
                               int64_t vunits, int ntouch, int n_new, int L, int D, int pos0, uint8_t* k_cache,
                               uint8_t* k_sc, uint8_t* v_cache, uint8_t* v_sc) {
  if ((int)blockIdx.x < kgroups) {
    kv_append_k_part((const float*)k_new, (int64_t)blockIdx.x * blockDim.x + threadIdx.x, kblocks, n_new, L, D, pos0,
                     k_cache, k_sc);
  } else {
    // (the workgroup's branch is uniform: the E3M2 table is filled by all its threads)
    __shared__ uint8_t e3m2_tab[FMT == 0 ? 4 : E3M2_TAB_N];
    if constexpr (FMT != 0) {
      e3m2_tab_fill(e3m2_tab, threadIdx.x, blockDim.x);
      __syncthreads();
    }
    const int64_t unit = ((int64_t)blockIdx.x - kgroups) * (blockDim.x / 64) + (threadIdx.x >> 6);
    kv_append_v_part<FMT>(v_new, v_tail, unit, vunits, threadIdx.x & 63, ntouch, n_new, L, D, pos0, v_cache, v_sc,
                          e3m2_tab);
  }
}

#define MXFA_KV_APPEND(FMT, NAME)                                                                             \
  extern "C" __global__ void __launch_bounds__(256)                                                          \
      NAME(const float* k_new, const float* v_new, float* v_tail, int64_t kblocks, int kgroups, int64_t vunits, \
           int ntouch, int n_new, int L, int D, int pos0, uint8_t* k_cache, uint8_t* k_sc, uint8_t* v_cache,   \
           uint8_t* v_sc) {                                                                                    \
    kv_append_impl<FMT>(k_new, v_new, v_tail, kblocks, kgroups, vunits, ntouch, n_new, L, D, pos0, k_cache, k_sc, \
                        v_cache, v_sc);                                                                        \
  }
MXFA_KV_APPEND(0, mxfa_kv_append_e4m3)
MXFA_KV_APPEND(1, mxfa_kv_append_e3m2)
MXFA_KV_APPEND(2, mxfa_kv_append_e3m2_blk)

// Tail of the block left open by an append that spans several blocks: rows of positions
// pos0 .. end - 1 from the new tokens, rows past the end zeroed (the block starts after
// pos0, so it holds no earlier rows).  One thread per (b * Hkv + kvh, row, 4 columns).
extern "C" __global__ void __launch_bounds__(256) mxfa_kv_tail_update(const float* v_new, float* v_tail,
                                                                      int64_t nthreads, int n_new, int D, int pos0) {
  const int64_t gt = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gt >= nthreads) return;
  const int cg = D / 4;
  const int64_t bk = gt / (32 * cg);
  const int rem = (int)(gt % (32 * cg));
  const int r = rem / cg, c4 = (rem % cg) * 4;
  const int end = pos0 + n_new;
  const int p = ((end - 1) / 32) * 32 + r;
  const float4 x = p < end ? *reinterpret_cast<const float4*>(v_new + (bk * n_new + (p - pos0)) * D + c4)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
  *reinterpret_cast<float4*>(v_tail + (bk * 32 + r) * D + c4) = x;
}

// ============================================================================
// Synthetic inputs: x[i] ~ N(0,1) from a counter-based hash (splitmix64) and
// Box-Muller; each element independently multiplied by `mul` with probability p.
// ============================================================================
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
  z += 0x9e3779b97f4a7c15ull;
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

extern "C" __global__ void __launch_bounds__(256) mxfa_fill_normal_f32(float* x, int64_t n, uint64_t seed,
                                                                       float outlier_p, float outlier_mul) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  uint64_t h = splitmix64(seed * 0x2545f4914f6cdd1dull + (uint64_t)i);
  float u1 = ((float)(uint32_t)(h >> 40) + 0.5f) * (1.0f / 16777216.0f);
  float u2 = (float)(uint32_t)((h >> 16) & 0xffffffu) * (1.0f / 16777216.0f);
  float r = sqrtf(-2.0f * logf(u1));
  float z = r * cosf(6.283185307179586f * u2);
  if (outlier_p > 0.0f) {
    uint64_t h2 = splitmix64(h ^ 0xa0761d6478bd642full);
    float u3 = (float)(uint32_t)(h2 >> 40) * (1.0f / 16777216.0f);
    if (u3 < outlier_p) z *= outlier_mul;
  }
  x[i] = z;
}
