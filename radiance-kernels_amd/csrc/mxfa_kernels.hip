// MXFP8 flash attention for MI355X (gfx950): quantizers, prefill, split-KV decode.
//
// Built with `hipcc --genco --offload-arch=gfx950` into mxfa_kernels.hsaco and
// launched by mxfa_host.cpp through hipModuleLaunchKernel.  Every entry point is
// extern "C" so the host looks it up by name.
//
// Reference path (ucb-bar/radiance-kernels): kernels/flash_attention_mx{,_gqa,
// _gemma,_fp6,_stable}.  Per key block the reference runs QK^T on the MX mesh,
// an online softmax + MX requant of P on the SIMT cores, then PV on the mesh and
// a rescale of the O accumulator (kernels/flash_attention_mx_gqa/kernel.cpp:124-175,
// flash_mx_impl.hpp:315-553).  Here PV runs on the scaled MXFP8 MFMA
// (v_mfma_scale_f32_32x32x64_f8f6f4), QK^T on the bf16 MFMA from an exact dequantization
// of the MX operands (see "Precision" below), and the softmax/requant on the VALU.
//
// Scaled-MFMA operand layout (32x32x64, fp8), measured on gfx950:
//   A (32 rows x 64 k): lane l holds row l%32; byte j of its 32 bytes is
//       k = 32*(j/16) + 16*(l/32) + j%16; the lane's scale applies to row l%32,
//       k-block l/32 (k in [32*(l/32), 32*(l/32)+32)).
//   B (64 k x 32 cols): lane l holds col l%32, same k mapping and scale rule.
//   C (32x32 fp32): lane l, reg i -> col l%32, row 8*(i/4) + 4*(l/32) + i%4.
// Attention computes S^T = K Q^T so a lane owns one query and 16 keys of every
// 32-key tile, which makes the per-(query, 32 keys) P scale a lane-pair
// reduction; O^T += V^T P^T then takes P straight from registers (B) and V^T
// from LDS through ds_read_b64_tr_b8 (A), with the key order of both operands
// matched to the S^T register order.
//
// Precision.  The scaled fp8 MFMA sums each group of 8 products in a fixed-point
// window of 14 significant bits below the group's largest product (measured on
// gfx950), so scores carry ~1e-3 relative error; R1's floor(log2(amax)) P scale
// turns such perturbations into whole-block requantization changes.  The scores
// are therefore computed on the bf16 MFMA (v_mfma_f32_32x32x16_bf16, fp32-exact
// accumulation) from the MX operands dequantized exactly into bf16 (E4M3 x 2^k is a
// bf16 value), while PV -- whose P operand is MX-quantized by definition -- runs on
// the scaled MXFP8 MFMA.  bf16 MFMA layout (32x32x16): lane l holds row/col l%32,
// k = 8*(l/32) + j for its 8 elements; C as above.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>
#include <utility>

#include "mx_device.h"
#include "mxfa_args.h"

using namespace mxfa;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) v2i lds_v2i;

#define LOG2E_F 1.4426950408889634f

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

// ============================================================================
// Attention
// ============================================================================
// FaArgs: see mxfa_args.h


constexpr int BN = 64;          // online-softmax key block (the reference's Bk)
constexpr int NWAVE = 4;

// Combine a value across the lane pair (l, l ^ 32) with v_permlane32_swap (no LDS):
// swap(x, x) returns (x of lanes 0-31 | x of lanes 0-31 moved up, x of lanes 32-63 moved
// down | x of lanes 32-63), so both halves hold their own and their partner's value.
__device__ __forceinline__ float pair_max(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ v16f mfma_mx(v8i a, v8i b, v16f c, int sa, int sb) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, sa, 0, sb);
}
// A operand in E5M2 (cbsz = 1), B in E4M3
__device__ __forceinline__ v16f mfma_mx_a5(v8i a, v8i b, v16f c, int sa, int sb) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 1, 0, 0, sa, 0, sb);
}
// A operand in fp6 E3M2 (cbsz = 3: lane l holds row l % 32 and k = 32 (l / 32) + i, element i
// in bits 6i .. 6i + 5 of dwords 0-5, measured on gfx950), B in E4M3
__device__ __forceinline__ v16f mfma_mx_a6(v8i a, v8i b, v16f c, int sa, int sb) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 3, 0, 0, sa, 0, sb);
}

__device__ __forceinline__ v16f mfma_bf16(v4i a, v4i b, v16f c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c, 0, 0, 0);
}

// 8 E4M3 codes (two dwords) x 2^(sc-127) -> 8 bf16 (exact), in element order.
__device__ __forceinline__ v4i fp8x8_to_bf16x8(uint32_t w0, uint32_t w1, float scale) {
  v4i o;
  o[0] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, scale, false));
  o[1] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w0, scale, true));
  o[2] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, scale, false));
  o[3] = __builtin_bit_cast(int, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w1, scale, true));
  return o;
}

// E8M0 code -> the float whose exponent field carries it (the scaled-convert operand).
__device__ __forceinline__ float e8m0_as_float(uint32_t code) { return __uint_as_float(code << 23); }

__device__ __forceinline__ v8i cat44(v4i lo, v4i hi) {
  return (v8i){lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Decode LDS slots: a 64-key block of fp8 codes (K, then V) at row pitch D + 16 bytes,
// whose 16-byte pad keeps row starts on distinct banks, and the block's V scales.
template <int D> struct Lds {
  static constexpr int KP = D + 16;          // V row pitch (bytes)
  static constexpr int TILE = BN * KP;
  static constexpr int SC = BN * D / 32;
};

// Buffer resource over [base + off, base + off + bytes): loads beyond it return 0, so
// key rows >= Sk need no branch.  Word 3 = raw 32-bit data format (gfx9 buffer layout).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const uint8_t* base, int64_t off, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)(base + off), 0, (int)(bytes > 0 ? bytes : 0), 0x00020000);
}

// Per-wave online-softmax state and O accumulator for 32 query columns.
template <int D>
struct WaveState {
  v16f o[D / 32];
  float m;       // running max (in x units), per lane = per query
  float l;       // per-lane partial row sum (the partner lane holds the rest)
};

// Visible keys of one query row: [klo, khi] (khi < klo when none), folding the causal
// limit, the sliding window, seq_k and row validity.
__device__ __forceinline__ void key_limits(const FaArgs& a, int qpos, bool qvalid, int& klo, int& khi) {
  khi = a.Sk - 1;
  if (a.causal) khi = min(khi, qpos);
  klo = a.window > 0 ? max(0, qpos - a.window + 1) : 0;
  if (!qvalid) khi = -1;
}

// ---- softmax-requant of one P tile (the reference's fused_softmax_requant,
// kernels/flash_attention_mx_gqa/flash_mx_impl.hpp:315-394, with rule R1).
// Scale: the tile amax is exp2((tile max - m) * c) -- exactly 1 in the tile holding
// the row max, like the reference's exp(S - m) -- and sc its R1 code.  P =
// exp2(fma(s, c, -m*c)); fma and exp2 are monotone, so no P of the tile exceeds the amax
// by more than one rounding residue, which leaves its code unchanged.
__device__ __forceinline__ uint32_t p_tile_scale(float bmax, float mu, float c) {
  return scale_code_p_fast(__builtin_amdgcn_exp2f((bmax - mu) * c));
}

// 16 P values of one lane: writes P and the codes (w[g] byte j = value 4g + j), adds
// the P values to lsum in order.
__device__ __forceinline__ void p_tile16(const v16f& s, float c, float mcn, uint32_t sc, float (&p)[16],
                                         uint32_t (&w)[4], float& lsum) {
#pragma unroll
  for (int i = 0; i < 16; i++) {
    p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[i], c, mcn));
    lsum += p[i];
  }
  const PTileBounds bnd = p_tile_bounds(sc);
#pragma unroll
  for (int g = 0; g < 4; g++) w[g] = p_pack4(p[4 * g], p[4 * g + 1], p[4 * g + 2], p[4 * g + 3], bnd);
}

// The same step with rule R2: P rounded to bf16 (the P written and summed), the scale
// from the bf16 tile amax, codes by mantissa truncation.
__device__ __forceinline__ uint32_t p_tile_scale_r2(float bmax, float mu, float c) {
  return r2_scale_code(__builtin_amdgcn_exp2f((bmax - mu) * c));
}

__device__ __forceinline__ void p_tile16_r2(const v16f& s, float c, float mcn, uint32_t sc, float (&p)[16],
                                            uint32_t (&w)[4], float& lsum) {
  const PTileR2 bnd = p_tile_r2(sc);
  float y[16];
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const uint32_t pb = bf16_rne_bits(__builtin_amdgcn_exp2f(__builtin_fmaf(s[i], c, mcn)));
    p[i] = __uint_as_float(pb);
    lsum += p[i];
    y[i] = r2_cut(pb, bnd);
  }
#pragma unroll
  for (int g = 0; g < 4; g++) w[g] = cvt_pack4(y[4 * g], y[4 * g + 1], y[4 * g + 2], y[4 * g + 3], bnd.scale);
}

// P rules of the attention kernels (template argument PR).
enum { P_R1 = 0, P_R2 = 1 };

template <int PR>
__device__ __forceinline__ uint32_t p_scale(float bmax, float mu, float c) {
  return PR == P_R2 ? p_tile_scale_r2(bmax, mu, c) : p_tile_scale(bmax, mu, c);
}

template <int PR>
__device__ __forceinline__ void p_tile(const v16f& s, float c, float mcn, uint32_t sc, float (&p)[16],
                                       uint32_t (&w)[4], float& lsum) {
  if constexpr (PR == P_R2)
    p_tile16_r2(s, c, mcn, sc, p, w, lsum);
  else
    p_tile16(s, c, mcn, sc, p, w, lsum);
}

// Test entry: the routine above on caller scores, one thread per row, 32-blocks along
// the row.  Outputs P, codes, scales, and the row sums of P.
template <int PR>
__device__ void softmax_requant_rows(const float* s, const float* row_max, float c, int64_t rows, int cols, float* p,
                                     uint8_t* codes, uint8_t* scales, float* row_sum) {
  const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= rows) return;
  const float mu = row_max[r], mcn = -(mu * c);
  float lsum = 0.0f;
  for (int j = 0; j < cols / 32; j++) {
    const int64_t off = r * cols + 32 * j;
    v16f a, b;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      float4 x = reinterpret_cast<const float4*>(s + off)[i];
      float4 y = reinterpret_cast<const float4*>(s + off)[4 + i];
      a[4 * i] = x.x; a[4 * i + 1] = x.y; a[4 * i + 2] = x.z; a[4 * i + 3] = x.w;
      b[4 * i] = y.x; b[4 * i + 1] = y.y; b[4 * i + 2] = y.z; b[4 * i + 3] = y.w;
    }
    float bmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; i++) bmax = fmaxf(bmax, fmaxf(a[i], b[i]));
    const uint32_t sc = p_scale<PR>(bmax, mu, c);
    float pa[16], pb[16];
    uint32_t wa[4], wb[4];
    p_tile<PR>(a, c, mcn, sc, pa, wa, lsum);
    p_tile<PR>(b, c, mcn, sc, pb, wb, lsum);
#pragma unroll
    for (int i = 0; i < 16; i++) {
      p[off + i] = pa[i];
      p[off + 16 + i] = pb[i];
    }
#pragma unroll
    for (int g = 0; g < 4; g++) {
      reinterpret_cast<uint32_t*>(codes + off)[g] = wa[g];
      reinterpret_cast<uint32_t*>(codes + off)[4 + g] = wb[g];
    }
    scales[r * (cols / 32) + j] = (uint8_t)sc;
  }
  row_sum[r] = lsum;
}

extern "C" __global__ void __launch_bounds__(256) mxfa_softmax_requant_rows(
    const float* s, const float* row_max, float c, int64_t rows, int cols, float* p, uint8_t* codes,
    uint8_t* scales, float* row_sum, int p_rule) {
  if (p_rule == P_R2)
    softmax_requant_rows<P_R2>(s, row_max, c, rows, cols, p, codes, scales, row_sum);
  else
    softmax_requant_rows<P_R1>(s, row_max, c, rows, cols, p, codes, scales, row_sum);
}

// Softmax, P requant and O^T += V^T P^T for one key block whose scores are in s.
// mask: the block has keys outside [klo, khi] for some row of the wave (wave-uniform).
// VBLK: the V tile is block-packed E3M2 as the caller stores it (two 32-key blocks of D
// columns x 24 bytes), read as the fp6 operand; else E4M3 codes [key][KP].
template <int D, bool SOFTCAP, int PR, bool VBLK = false>
__device__ __forceinline__ void softmax_pv(WaveState<D>& st, v16f (&s)[BN / 32], const uint8_t* sV,
                                           const uint8_t* sVs, int key0, int klo, int khi, bool mask,
                                           const FaArgs& a, int lane) {
  constexpr int KP = Lds<D>::KP;
  constexpr int NT = BN / 32;
  const int r = lane & 31, h = lane >> 5;

  // ---- scores in log2 units (softcap) or raw units, masked -> -inf
  if (SOFTCAP) {
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
      for (int i = 0; i < 16; i++) {
        float u = s[t][i] * a.sc_u;
        float e = __builtin_amdgcn_exp2f(-2.0f * LOG2E_F * fabsf(u));
        float th = (1.0f - e) * __builtin_amdgcn_rcpf(1.0f + e);
        s[t][i] = a.cap_log2 * (u < 0.0f ? -th : th);
      }
  }
  if (mask) {
    // The empty asm keeps this pass behind the (wave-uniform) branch: without it the
    // selects are speculated into every block.
    __asm__ volatile("");
    const int dhi = khi - key0 - 4 * h, dlo = klo - key0 - 4 * h;
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
      for (int i = 0; i < 16; i++) {
        // kpos - key0 - 4h is a compile-time constant per (t, i): two compares per element
        const int c = 32 * t + 8 * (i >> 2) + (i & 3);
        s[t][i] = ((c <= dhi) & (c >= dlo)) ? s[t][i] : -INFINITY;
      }
  }
  float tmax[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) {
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; i++) mx = fmaxf(mx, s[t][i]);
    tmax[t] = mx;
  }
  // block (query, 32-key tile) maxima: combine the lane pair (l, l^32)
  float bmax[NT];
  float rmax = -INFINITY;
#pragma unroll
  for (int t = 0; t < NT; t++) {
    bmax[t] = pair_max(tmax[t]);
    rmax = fmaxf(rmax, bmax[t]);
  }
  // The row maximum must give a block amax of exactly exp2(0) = 1, like the reference's
  // exp(S - m): a fused x*c - m*c would leave a rounding residue that can move that
  // block's power-of-two scale, so the amax below uses (max - m) * c.
  const float c = SOFTCAP ? 1.0f : a.c_log2;
  float m_new = fmaxf(st.m, rmax);
  float mu = m_new == -INFINITY ? 0.0f : m_new;
  float corr = st.m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((st.m - mu) * c);
  st.m = m_new;

  // ---- P tiles: scale from the exact tile amax, R1 (or R2) codes
  const float mcn = -(mu * c);
  float lsum = 0.0f;
  v8i pb[NT / 2];                    // P codes: B operand of each 64-key PV step
  int psc[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const uint32_t sc = p_scale<PR>(bmax[t], mu, c);
    psc[t] = (int)sc;
    float p[16];
    uint32_t w[4];
    p_tile<PR>(s[t], c, mcn, sc, p, w, lsum);
#pragma unroll
    for (int g = 0; g < 4; g++) pb[t >> 1][4 * (t & 1) + g] = (int)w[g];
  }
  st.l = st.l * corr + lsum;

  // ---- O^T = O^T * corr + V^T P^T (the rescale is skipped when no query of the wave
  // raised its max: corr == 1 exactly and the product would be the identity)
  if (__any(corr != 1.0f)) {
#pragma unroll
    for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
      for (int i = 0; i < 16; i++) st.o[dt][i] *= corr;
  }

  if constexpr (VBLK) {
    static_assert(BN == 64, "one 64-key PV step");
    // lane (d, h) reads the 24 bytes of column 32 dt + r of 32-key block h: three ds_read_b64,
    // lanes 24 bytes apart (32 distinct even banks)
    const int pscale = psc[h];
    const uint8_t* a0 = sV + h * (24 * D) + 24 * r;
#pragma unroll
    for (int dt = 0; dt < D / 32; dt++) {
      const v2i* src = reinterpret_cast<const v2i*>(a0 + 768 * dt);
      const v2i x0 = src[0], x1 = src[1], x2 = src[2];
      const v8i va = (v8i){x0[0], x0[1], x1[0], x1[1], x2[0], x2[1], 0, 0};
      st.o[dt] = mfma_mx_a6(va, pb[0], st.o[dt], sVs[h * D + dt * 32 + r], pscale);
    }
    return;
  }
  const int l16 = lane & 15, g16 = lane >> 4;
#pragma unroll
  for (int kstep = 0; kstep < BN / 64; kstep++) {
    int pscale = psc[2 * kstep + h];
#pragma unroll
    for (int dt = 0; dt < D / 32; dt++) {
      v8i va;
      // byte t of read q: key 64*kstep + 32*(q/2) + 16*(q%2) + 8*(t/4) + 4*h + t%4, d = 32*dt + lane%32
      const int t8 = l16 >> 1;
      const int dcol = dt * 32 + 16 * (g16 & 1) + 8 * (l16 & 1);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        int key = 64 * kstep + 32 * (q >> 1) + 16 * (q & 1) + 8 * (t8 >> 2) + 4 * h + (t8 & 3);
        v2i rv = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(sV + key * KP + dcol));
        va[2 * q] = rv[0];
        va[2 * q + 1] = rv[1];
      }
      int vscale = sVs[(2 * kstep + h) * D + dt * 32 + r];
      st.o[dt] = mfma_mx(va, pb[kstep], st.o[dt], vscale, pscale);
    }
  }
}

// Q operand (B of S^T = K Q^T, bf16) for query row `qrow` (zeros if invalid): MFMA kk
// takes d = 16*kk + 8*h .. +7, dequantized with the row's E8M0 scale of that 32-block.
template <int D>
__device__ __forceinline__ void load_q(v4i* qb, const uint8_t* qrow, const uint8_t* qsrow, bool valid, int h) {
#pragma unroll
  for (int kk = 0; kk < D / 16; kk++) {
    v4i o = {0, 0, 0, 0};
    if (valid) {
      v2i w = *reinterpret_cast<const v2i*>(qrow + 16 * kk + 8 * h);
      o = fp8x8_to_bf16x8((uint32_t)w[0], (uint32_t)w[1], e8m0_as_float(qsrow[kk / 2]));
    }
    qb[kk] = o;
  }
}

// Split-d operand mapping of the decode kernels: lane half h owns d in [h*D/2, (h+1)*D/2)
// and MFMA kk takes d = h*D/2 + 8*kk .. +7 (any d-to-k assignment gives the same dot
// product when Q and K use it alike).  A lane's K operand is then one contiguous
// half-row of the key, read straight from global memory.
template <int D>
__device__ __forceinline__ void load_q_split(v4i* qb, const uint8_t* qrow, const uint8_t* qsrow, bool valid, int h) {
#pragma unroll
  for (int kk = 0; kk < D / 16; kk++) {
    const int d0 = h * (D / 2) + 8 * kk;
    v4i o = {0, 0, 0, 0};
    if (valid) {
      v2i w = *reinterpret_cast<const v2i*>(qrow + d0);
      o = fp8x8_to_bf16x8((uint32_t)w[0], (uint32_t)w[1], e8m0_as_float(qsrow[d0 / 32]));
    }
    qb[kk] = o;
  }
}


// ---------------------------------------------------------------------------
// LDS helpers of the prefill kernels: the V tile swizzle, LDS addresses, LDS DMA.
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void lds_void;

// 16-byte chunk c of V key row `key` sits at chunk c ^ vsw(key) of its row: the
// ds_read_b64_tr_b8 reads of the PV operand (16 keys x 32 bytes per instruction) then hit
// distinct banks, with no row padding (so a 1 KB DMA instruction fills whole rows).
template <int D> __device__ __forceinline__ int vsw(int key) {
  if constexpr (D == 256) return 2 * ((key & 3) | (((key >> 3) & 1) << 2));   // rows alias all 64 banks
  return D == 128 ? 2 * (((key >> 1) & 1) | ((key >> 2) & 2)) : ((key & 1) | (((key >> 3) & 1) << 1));
}

// A generic pointer into LDS -> the LDS address (its low 32 bits), without the aperture
// check a generic-to-local cast would emit.
__device__ __forceinline__ lds_void* lds_addr(const void* p) {
  return (lds_void*)(uint32_t)(uintptr_t)p;
}

// soff: a wave-uniform byte offset added to the source address (not to the LDS address)
template <int SIZE>
__device__ __forceinline__ void dma_lds(__amdgpu_buffer_rsrc_t r, uint8_t* lds_base, int voff, int soff = 0) {
  if constexpr (SIZE == 16)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds_addr(lds_base), 16, voff, soff, 0, 0);
  else if constexpr (SIZE == 4)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds_addr(lds_base), 4, voff, soff, 0, 0);
  else
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, lds_addr(lds_base), 2, voff, soff, 0, 0);
}

// max(a, b) without the canonicalizing maxes fmaxf adds on operands the compiler cannot prove
// canonical (MFMA results, cross-lane swaps): IEEE maximum (v_maximum3_f32 on gfx950; a NaN
// score, possible only from NaN operand codes, propagates instead of being dropped).
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// max of the 16 scores of one S^T tile held by a lane
__device__ __forceinline__ float tile_max16(const v16f& x) {
  float m = vmax(x[0], x[1]);
#pragma unroll
  for (int i = 2; i < 16; i++) m = vmax(m, x[i]);
  return m;
}

// A wave-uniform value in a VGPR: VALU instructions whose operands are all VGPRs issue at
// the full rate, one with a scalar operand at half of it.
__device__ __forceinline__ float in_vgpr(float x) {
  float r;
  __asm__("v_mov_b32 %0, %1" : "=v"(r) : "s"(x));
  return r;
}
__device__ __forceinline__ uint32_t in_vgpr_u(uint32_t x) {
  uint32_t r;
  __asm__("v_mov_b32 %0, %1" : "=v"(r) : "s"(x));
  return r;
}

// fp32 subnormal results flushed to zero (MODE.FP_DENORM single-precision bits = 0) for the
// rest of the wave.  The pipelined prefill kernels rely on it for the R1 flush of P (below);
// elsewhere it only turns results below 2^-126 into zeros.
__device__ __forceinline__ void fp32_flush_denormals() {
  __builtin_amdgcn_s_setreg((1 << 11) | (4 << 6) | 1, 0);   // hwreg(MODE, 4, 2)
}

__device__ __forceinline__ float pair_max_raw(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// R1 codes of four P values of a tile with scale code sc, given y = P * 2^(7 - sc) computed
// with fp32 subnormals flushed (fp32_flush_denormals): the R1 flush bound of the tile,
// F4M3 * 2^(sc - 127), is within two ulps below 2^(sc - 133), the bound that the flush to zero
// applies (y < 2^-126), and no exponential lands in between: sc <= 119 (amax <= 1), so
// P = exp2(x) with x within 2^-19 of an integer e <= -14 is 2^e itself or at least ~10 ulps
// from it.  The kept values convert as y * 2^120 = P / 2^(sc - 127), the same codes.
__device__ __forceinline__ uint32_t p_pack4_ftz(float y0, float y1, float y2, float y3, uint32_t ones) {
  const uint32_t w = cvt_pack4_in_place(y0, y1, y2, y3, __uint_as_float(7u << 23));   // 2^-120
  const uint32_t top = (w + ones) >> 7;               // bit 0 of each byte: that byte was 0x7f
  return w ^ (top & ones);                            // 0x7f -> 0x7e, other bytes unchanged
}

__device__ __forceinline__ float vmin(float a, float b) { return __builtin_elementwise_minimum(a, b); }
__device__ __forceinline__ float tile_min16(const v16f& x) {
  float m = vmin(x[0], x[1]);
#pragma unroll
  for (int i = 2; i < 16; i++) m = vmin(m, x[i]);
  return m;
}
__device__ __forceinline__ float pair_min_raw(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return vmin(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// With a softcap, s holds r = 1 / (e + 1) per score (pipe_scores; masked keys r = +inf) and
// the capped score is cap + cap2 * r (cap2 = -2 cap < 0, cap = softcap * log2(e)): the
// exponent's argument is fma(cap2, r, cap - mu), one operation like fma(s, c, -mu * c)
// without a softcap.  The score is non-increasing in r (fma rounds monotonically), so the
// tile maximum is cap + cap2 * min(r), bit for bit the maximum of the capped scores, and
// -inf for a fully masked tile (cap2 * inf).
// VG: the softcap constants in VGPRs (full-rate VALU at three waves per SIMD); at two waves
// per SIMD SGPR operands cost nothing and save the registers.
template <bool SOFTCAP, int PR, bool VG = true>
__device__ __forceinline__ void pipe_softmax(float& m, float& l, v16f (&s)[BN / 32],
                                             v8i& pb, int (&psc)[BN / 32], float& corr, float c,
                                             float cap2 = 0.0f, float cap = 0.0f) {
  constexpr int NT = BN / 32;
  if (SOFTCAP && VG) {
    cap2 = in_vgpr(cap2);
    cap = in_vgpr(cap);
  }
  float bmax[NT];
#pragma unroll
  for (int t = 0; t < NT; t++)
    bmax[t] = SOFTCAP ? __builtin_fmaf(cap2, pair_min_raw(tile_min16(s[t])), cap) : pair_max_raw(tile_max16(s[t]));
  float rmax = bmax[0];
#pragma unroll
  for (int t = 1; t < NT; t++) rmax = vmax(rmax, bmax[t]);
  const float m_new = vmax(m, rmax);
  const float mu = m_new == -INFINITY ? 0.0f : m_new;
  corr = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((m - mu) * c);
  m = m_new;
  const float mcn = SOFTCAP ? cap - mu : -(mu * c);
  auto arg = [&](float x) { return SOFTCAP ? __builtin_fmaf(cap2, x, mcn) : __builtin_fmaf(x, c, mcn); };
  float part[4];
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const float amax = __builtin_amdgcn_exp2f((bmax[t] - mu) * c);
    uint32_t sc;
    if constexpr (PR == P_R2)
      sc = r2_scale_code(amax);
    else
      sc = scale_code_p_nb(amax);
    psc[t] = (int)sc;
    float p[16];
    uint32_t w[4];
    if constexpr (PR == P_R2) {
      const PTileR2 bnd = p_tile_r2(sc);
      float y[16];
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const uint32_t pbits = bf16_rne_bits(__builtin_amdgcn_exp2f(arg(s[t][i])));
        p[i] = __uint_as_float(pbits);
        y[i] = r2_cut(pbits, bnd);
      }
#pragma unroll
      for (int g = 0; g < 4; g++) w[g] = cvt_pack4(y[4 * g], y[4 * g + 1], y[4 * g + 2], y[4 * g + 3], bnd.scale);
    } else {
#pragma unroll
      for (int i = 0; i < 16; i++) p[i] = __builtin_amdgcn_exp2f(arg(s[t][i]));
      const float f = __uint_as_float((134u - sc) << 23);     // 2^(7 - sc)
      const uint32_t ones = in_vgpr_u(0x01010101u);
#pragma unroll
      for (int g = 0; g < 4; g++)
        w[g] = p_pack4_ftz(p[4 * g] * f, p[4 * g + 1] * f, p[4 * g + 2] * f, p[4 * g + 3] * f, ones);
    }
    // row-sum terms (every P, including those R1 flushes from the codes) in four
    // independent chains (no 32-deep add dependency)
#pragma unroll
    for (int i = 0; i < 16; i++) part[i & 3] = (t == 0 && i < 4) ? p[i] : part[i & 3] + p[i];
#pragma unroll
    for (int g = 0; g < 4; g++) pb[4 * (t & 1) + g] = (int)w[g];
  }
  l = l * corr + ((part[0] + part[1]) + (part[2] + part[3]));
}
// Score post-processing of one block in place: softcap (log2 units), then the mask.
// softcap * tanh(u), u = s * scale / softcap, in log2 units: cap_log2 * (1 - 2 / (e + 1)) =
// cap_log2 + cap2 * r with e = exp2(2 log2(e) u), r = 1 / (e + 1), cap2 = -2 cap_log2.  s keeps
// r (an exponential and a reciprocal per score); pipe_softmax applies cap_log2 + cap2 * r
// inside the exponential's argument.  e = inf and e = 0 give +-cap_log2 exactly.
// VG: the constant in a VGPR (full-rate VALU at three waves per SIMD; at two waves an SGPR
// operand costs nothing and saves the register).
template <bool SOFTCAP, bool VG = true>
__device__ __forceinline__ void pipe_scores(v16f (&s)[BN / 32], const FaArgs& a) {
  if (SOFTCAP) {
    float k2 = 2.0f * LOG2E_F * a.sc_u;
    if (VG) k2 = in_vgpr(k2);
#pragma unroll
    for (int t = 0; t < BN / 32; t++)
#pragma unroll
      for (int i = 0; i < 16; i++) s[t][i] = __builtin_amdgcn_rcpf(__builtin_amdgcn_exp2f(s[t][i] * k2) + 1.0f);
  }
}

// The capped score of a softcap block's entry r (for the stage trace).
__device__ __forceinline__ float capped_score(float r, const FaArgs& a) {
  return __builtin_fmaf(-2.0f * a.cap_log2, r, a.cap_log2);
}

// Masked keys get -inf, or with a softcap r = +inf (capped score cap + cap2 * inf = -inf).
template <bool SOFTCAP>
__device__ __forceinline__ void pipe_mask(v16f (&s)[BN / 32], int key0, int klo, int khi, int h) {
  const int dhi = khi - key0 - 4 * h, dlo = klo - key0 - 4 * h;
  constexpr float masked = SOFTCAP ? INFINITY : -INFINITY;
#pragma unroll
  for (int t = 0; t < BN / 32; t++)
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const int c = 32 * t + 8 * (i >> 2) + (i & 3);
      s[t][i] = ((c <= dhi) & (c >= dlo)) ? s[t][i] : masked;
    }
}

// PV of one block in NP parts of D / NP columns: the operand registers of one part at a time
// (D = 256 at two waves per SIMD: 32 registers instead of 64).
template <int D, int NP, bool V5 = false>
__device__ __forceinline__ void pv_parts(v16f (&o)[D / 32], const uint8_t* sv, const v8i& pb, const int (&psc)[BN / 32],
                                         int lane) {
  constexpr int NT = D / 32 / NP;
  const int r = lane & 31, h = lane >> 5;
  const int l16 = lane & 15, g16 = lane >> 4;
  const int t8 = l16 >> 1;
  const int kl = 8 * (t8 >> 2) + 4 * h + (t8 & 3);
  const int sg = (g16 & 1) ^ vsw<D>(kl);
  // the lane's row scale of its key half, psc[h], by arithmetic (a select of the two array
  // elements becomes an indexed load of a private array)
  const int hmask = -(int)__builtin_amdgcn_ubfe((uint32_t)lane, 5, 1);
  const int pscale = psc[0] ^ ((psc[0] ^ psc[1]) & hmask);
  // d tile dt's operand address: the chunk index 2dt ^ sg is 16-byte granular, and the
  // row offset kl * D sets no bit below 6 (D = 64) or 7 / 8, so over a tile aligned to 256
  // bytes the LDS address is addr(0) ^ 32 dt
  const uint32_t a0 = (uint32_t)(uintptr_t)lds_addr(sv) + kl * D + (sg << 4) + 8 * (l16 & 1);
#pragma unroll
  for (int part = 0; part < NP; part++) {
    v8i va[NT];
    int vs[NT];
#pragma unroll
    for (int u = 0; u < NT; u++) {
      const int dt = part * NT + u;
      const uint32_t base = a0 ^ (uint32_t)(32 * dt);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const v2i rv = __builtin_amdgcn_ds_read_tr8_b64_v2i32(
            (lds_v2i*)(uintptr_t)(base + (32 * (q >> 1) + 16 * (q & 1)) * D));
        va[u][2 * q] = rv[0];
        va[u][2 * q + 1] = rv[1];
      }
      vs[u] = sv[BN * D + h * D + dt * 32 + r];   // the V scales follow the BN x D codes
    }
#pragma unroll
    for (int u = 0; u < NT; u++)
      o[part * NT + u] = V5 ? mfma_mx_a5(va[u], pb, o[part * NT + u], vs[u], pscale)
                            : mfma_mx(va[u], pb, o[part * NT + u], vs[u], pscale);
    if (part + 1 < NP) __builtin_amdgcn_sched_barrier(0);
  }
}

// PV of one block with V in the E3M2 block-packed layout: the LDS tile holds, per 32-key block
// kb (0, 1) and d, the block's 24 bytes at kb * 24D + 24 d -- exactly the fp6 A operand of
// lane (d % 32) + 32 kb, read with three ds_read_b64 (lanes 24 bytes apart: 32 distinct
// even banks, conflict-free).  V scales follow at BN * D as for E4M3 V.
template <int D, int NP>
__device__ __forceinline__ void pv_parts_blk(v16f (&o)[D / 32], const uint8_t* sv, const v8i& pb,
                                             const int (&psc)[BN / 32], int lane) {
  constexpr int NT = D / 32 / NP;
  const int r = lane & 31, h = lane >> 5;
  const int hmask = -(int)__builtin_amdgcn_ubfe((uint32_t)lane, 5, 1);
  const int pscale = psc[0] ^ ((psc[0] ^ psc[1]) & hmask);
  const uint8_t* a0 = sv + h * (24 * D) + 24 * r;
#pragma unroll
  for (int part = 0; part < NP; part++) {
    v8i va[NT];
    int vs[NT];
#pragma unroll
    for (int u = 0; u < NT; u++) {
      const int dt = part * NT + u;
      const v2i* src = reinterpret_cast<const v2i*>(a0 + 768 * dt);
      const v2i x0 = src[0], x1 = src[1], x2 = src[2];
      va[u] = (v8i){x0[0], x0[1], x1[0], x1[1], x2[0], x2[1], 0, 0};
      vs[u] = sv[BN * D + h * D + dt * 32 + r];
    }
#pragma unroll
    for (int u = 0; u < NT; u++) o[part * NT + u] = mfma_mx_a6(va[u], pb, o[part * NT + u], vs[u], pscale);
    if (part + 1 < NP) __builtin_amdgcn_sched_barrier(0);
  }
}

// O of one wave (32 query rows x D, MFMA layout), normalized by inv, stored through LDS so
// that every store instruction writes whole 128-byte lines: a lane of the MFMA layout holds
// 16-byte pieces of its row 128 bytes apart, whose line-partial stores cost 20% extra HBM
// writes.  Per 64-column chunk the wave writes its 32 x 64 floats to its private 8 KB slice
// ldsw (the 16-byte chunk c of row r at c ^ (r & 15)), then reads 4 rows x 256 contiguous
// bytes per instruction and stores them non-temporally (O is not read again here, so K and V
// keep the L2).  Rows qw0 + row >= Sq are not stored.
template <int D>
__device__ __forceinline__ void store_o_lds(const v16f (&o)[D / 32], float inv, float* ldsw, float* obase, int qw0,
                                            int Sq, int lane) {
  const int r = lane & 31, h = lane >> 5;
#pragma unroll
  for (int p = 0; p < D / 64; p++) {
#pragma unroll
    for (int dd = 0; dd < 2; dd++)
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int dt = 2 * p + dd, cidx = dd * 8 + 2 * g + h;
        const float4 w = make_float4(o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv, o[dt][4 * g + 2] * inv,
                                     o[dt][4 * g + 3] * inv);
        *reinterpret_cast<float4*>(ldsw + r * 64 + ((cidx ^ (r & 15)) << 2)) = w;
      }
#pragma unroll
    for (int k = 0; k < 8; k++) {
      const int row = 4 * k + (lane >> 4), c = lane & 15;
      const float4 v = *reinterpret_cast<const float4*>(ldsw + row * 64 + ((c ^ (row & 15)) << 2));
      if (qw0 + row < Sq)
        __builtin_nontemporal_store(__builtin_bit_cast(v4i, v),
                                    reinterpret_cast<v4i*>(obase + (int64_t)(qw0 + row) * D + 64 * p + 4 * c));
    }
  }
}


// ---------------------------------------------------------------------------
// Prefill at three waves per SIMD (D <= 128, E4M3 V).  The MX K operand is dequantized
// once, by mxfa_k_to_bf16, into a bf16 copy [B][Hkv][Sk][D] (exact: E4M3 x 2^k is a bf16
// value); the prefill stages that copy and V into LDS by DMA, so it holds no staging
// registers and converts nothing: 168 registers per lane, three 4-wave workgroups per CU.
// With every wave issuing at most one instruction per few cycles, the third wave per SIMD
// raises the issue rate by half.  Per key block j, one barrier:
//   DMA K_bf16(j+1), V(j+1) into the other stage -> scores of j (bf16 MFMA) -> mask ->
//   softmax + P requant -> O rescale -> PV (scaled MXFP8 MFMA) -> wait, barrier.
// ---------------------------------------------------------------------------
// Workspace pre-pass: each thread converts PRE_G chunks of 16 codes (one 32-block half) of
// one (batch, KV head) -- blockIdx.y -- the workgroup's 256 * PRE_G consecutive chunks of
// that head, all loads issued before the stores (PRE_G = 8: 8.7 vs 10.2 us on the S = 4096
// GQA prefill, one workgroup per CU; 2 and 4 were slower).  D / 16 chunks per row (4, 8 or
// 16) divides 256, so a thread's chunks share one column and step 256 / (D / 16) rows.
// Row t of head h in the copies is row h * Skc + t of the cache-strided input: the bf16 value
// of K (kbf) and, when vws is set, the E4M3 code of E3M2 V (e3m2x4_to_e4m3x4: the same
// value) -- one launch for both.
constexpr int PRE_G = 8;
extern "C" __global__ void __launch_bounds__(256) mxfa_k_to_bf16(const uint8_t* __restrict__ k,
                                                                  const uint8_t* __restrict__ ks,
                                                                  const uint8_t* __restrict__ v, int D, int Sk,
                                                                  int Skc, uint8_t* __restrict__ kbf,
                                                                  uint8_t* __restrict__ vws) {
  const int lcpr = D == 256 ? 4 : D == 128 ? 3 : 2;
  const int c0 = blockIdx.x * blockDim.x * PRE_G + threadIdx.x;   // chunk within the head
  const int col = c0 & ((1 << lcpr) - 1);
  const int rstep = (int)blockDim.x >> lcpr;
  const int t0 = c0 >> lcpr;
  const int64_t hq = blockIdx.y;
  int64_t so[PRE_G], doff[PRE_G];   // source and copy byte offsets of chunk g (past the end: row 0)
  v4i x[PRE_G];
  float sc[PRE_G];
#pragma unroll
  for (int g = 0; g < PRE_G; g++) {
    const int t = t0 + g * rstep;
    const int64_t src = t < Sk ? hq * Skc + t : 0;
    so[g] = src * D + col * 16;
    doff[g] = (hq * Sk + t) * D + col * 16;
    x[g] = *reinterpret_cast<const v4i*>(k + so[g]);
    sc[g] = e8m0_as_float(ks[src * (D / 32) + col / 2]);
  }
#pragma unroll
  for (int g = 0; g < PRE_G; g++) {
    if (t0 + g * rstep < Sk) {
      v4i* o = reinterpret_cast<v4i*>(kbf + doff[g] * 2);
      o[0] = fp8x8_to_bf16x8((uint32_t)x[g][0], (uint32_t)x[g][1], sc[g]);
      o[1] = fp8x8_to_bf16x8((uint32_t)x[g][2], (uint32_t)x[g][3], sc[g]);
    }
  }
  if (vws) {
#pragma unroll
    for (int g = 0; g < PRE_G; g++) x[g] = *reinterpret_cast<const v4i*>(v + so[g]);
#pragma unroll
    for (int g = 0; g < PRE_G; g++) {
      if (t0 + g * rstep < Sk) {
        v4i z;
#pragma unroll
        for (int w = 0; w < 4; w++) z[w] = (int)e3m2x4_to_e4m3x4((uint32_t)x[g][w]);
        *reinterpret_cast<v4i*>(vws + doff[g]) = z;
      }
    }
  }
}

// bf16 K tile, chunk-major in groups of 16 rows: the 16-byte chunk c of key row `row` sits at
// (row / 16) * 32D + c * 256 + (row % 16) * 16.  A score-operand read (one chunk of 16
// consecutive rows per pass) covers 256 contiguous bytes -- all banks once -- and every
// read address is the lane's base plus an immediate; so are the DMA source offsets (each
// 1 KB DMA instruction fills 4 chunks of one 16-row group).
template <int D> struct P3Lds {
  static constexpr int KB = BN * 2 * D;           // bf16 K tile
  static constexpr int KDMA = KB / 1024;          // DMA instructions per K tile
  static constexpr int V = BN * D;                // V tile (16-byte chunks swizzled by vsw)
  static constexpr int VDMA = V / 1024;
  static constexpr int SCB = 2 * D > 256 ? 2 * D : 256;   // V scales [BN / 32][D], dword DMA
};

// Waves per prefill3 workgroup (4) and K stages: two for D <= 128 (three workgroups per CU);
// one for D = 256 (65 KB of tiles: two independent workgroups per CU, two waves per SIMD),
// whose next K block is brought in after every wave has read the current one.
template <int D> struct P3Waves { static constexpr int N = 4; };
template <int D> constexpr bool p3_one_k_stage() { return D == 256; }

// DMA of one key block into the prefill3 tiles by NW waves.  K: the four 16-row groups of the
// chunk-major tile, NW / 4 waves per group, each issuing 2D / 64 / (NW / 4) instructions of
// four 16-byte chunks per row (wave-uniform column offset as the scalar offset, within a
// row, so the range check sees the row either way).  V: VDMA / NW instructions per wave
// whose rows share the swizzle bits (p3_v_instr).  V scales: every wave issues the same dword
// instructions (same bytes), so the sequence has no branch.  The vector offsets are
// loop-invariant lane parts, the block and column offsets scalar offsets (P3Src).
struct P3Lane {
  int k, v, s;
};

// V DMA instruction m of wave w (1024 / D rows each).  The swizzle uses key bits 1 and 3
// (D = 128: instructions of equal parity), bits 0, 1, 3 (D = 256: equal bit 1) or bits 0
// and 3 (D = 64: within one instruction).
template <int D, int NW> __device__ __forceinline__ int p3_v_instr(int w, int m) {
  if constexpr (D == 128) return 4 * (w >> 1) + (w & 1) + 2 * m;                       // NW = 4
  else if constexpr (D == 256 && NW == 8) return 2 * w + m;
  else if constexpr (D == 256) return 2 * (w & 1) + 8 * (w >> 1) + (m & 1) + 4 * (m >> 1);   // NW = 4
  else return w + 4 * m;                                                                  // D = 64
}

template <int D, int NW> __device__ __forceinline__ P3Lane p3_lane(int wave, int lane) {
  constexpr unsigned VRPI = 1024 / D, CPR = D / 16, WPG = NW / 4, IPW = 2 * D / 64 / WPG;
  const unsigned ln = (unsigned)lane, w = (unsigned)wave;
  const unsigned vrow = (unsigned)p3_v_instr<D, NW>(wave, 0) * VRPI + ln / CPR, pos = ln % CPR;
  return {(int)((16 * (w / WPG) + ln % 16) * (2 * D) + (w % WPG) * IPW * 64 + (ln / 16) * 16),
          (int)(vrow * D + ((pos ^ (unsigned)vsw<D>((int)vrow)) << 4)), (int)(ln * 4)};
}

// Sources of the prefill3 DMA for one (b, KV head): buffer resources over the bf16 K rows
// (2D bytes each), the V codes (E4M3) and the V scales, each ending at key Sk.  The block
// and column offsets go in the loads' scalar offset, which the range check includes (measured
// on gfx950: a load whose vector offset is in range and whose scalar offset is not reads 0,
// for plain and LDS-DMA loads alike), so keys >= Sk still read 0.
struct P3Src {
  __amdgpu_buffer_rsrc_t k, v, vs;
};

__device__ __forceinline__ P3Src p3_src(const uint8_t* kbf, const uint8_t* v, const uint8_t* vs, int Sk, int D) {
  return {buf_rsrc(kbf, 0, (int64_t)Sk * (2 * D)), buf_rsrc(v, 0, (int64_t)Sk * D), buf_rsrc(vs, 0, (int64_t)(Sk / 32) * D)};
}

// V of block-packed E3M2 (VBLK): the block's two 32-key MX blocks are 48 D contiguous bytes
// of the caller's array (24 per (32-key block, d)), copied as they are by 3D / 64 one-KB
// instructions dealt to the waves in turn.
template <int D, int NW>
__device__ __forceinline__ void p3_dma_vblk(__amdgpu_buffer_rsrc_t rv, uint8_t* v, int key0, int wave, int lane) {
  constexpr int NV = 48 * D / 1024;
#pragma unroll
  for (int m = 0; m < (NV + NW - 1) / NW; m++) {
    const int i = wave + NW * m;
    if (NV % NW == 0 || i < NV) dma_lds<16>(rv, v + i * 1024, lane * 16, (key0 / 32) * (24 * D) + i * 1024);
  }
}

template <int D, int NW, bool DO_K = true, bool DO_V = true, bool VBLK = false>
__device__ __forceinline__ void p3_dma(const P3Src& src, uint8_t* kb, uint8_t* v, int key0, int wave, const P3Lane& pl,
                                       int lane = 0) {
  using L = P3Lds<D>;
  constexpr int WPG = NW / 4, IPW = 2 * D / 64 / WPG;   // waves per 16-row group, K instructions per wave
  constexpr int VPW = L::VDMA / NW;                     // V instructions per wave
  if constexpr (DO_K) {
    uint8_t* kdst = kb + (wave / WPG) * (32 * D) + (wave % WPG) * IPW * 1024;
#pragma unroll
    for (int m = 0; m < IPW; m++) dma_lds<16>(src.k, kdst + m * 1024, pl.k, key0 * (2 * D) + 64 * m);
  }
  if constexpr (DO_V && VBLK) p3_dma_vblk<D, NW>(src.v, v, key0, wave, lane);
  if constexpr (DO_V && !VBLK) {
    const int i0 = p3_v_instr<D, NW>(wave, 0);
#pragma unroll
    for (int m = 0; m < VPW; m++) {
      const int i = p3_v_instr<D, NW>(wave, m);
      dma_lds<16>(src.v, v + i * 1024, pl.v, key0 * D + (i - i0) * 1024);
    }
  }
  if constexpr (DO_V) {
#pragma unroll
    for (int m = 0; m < (2 * D + 255) / 256; m++) dma_lds<4>(src.vs, v + L::V + m * 256, pl.s, (key0 / 32) * D + m * 256);
  }
}

// Schedule of the score MFMAs with the next block's DMA: after the first two K operand
// reads, per MFMA one more read, two scalar instructions and a DMA instruction, so the wave
// issues the DMA while the matrix pipe works instead of before it.
template <int D>
__device__ __forceinline__ void p3_dma_interleave() {
  __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);      // DS reads
#pragma unroll
  for (int k = 0; k < D / 16 * (BN / 32); k++) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // MFMA
    __builtin_amdgcn_sched_group_barrier(0x004, 2, 0);    // SALU
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);    // VMEM read (LDS DMA)
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);    // DS read
  }
}

template <int D>
__device__ __forceinline__ void p3_qk(v16f (&s)[BN / 32], const v4i* qb, const uint8_t* kb, int lane) {
  const int r = lane & 31, h = lane >> 5;
  // row t*32 + r, chunk 2kk + h
  const uint8_t* kbase = kb + (r / 16) * (32 * D) + h * 256 + (r % 16) * 16;
#pragma unroll
  for (int t = 0; t < BN / 32; t++) s[t] = (v16f){};
#pragma unroll
  for (int kk = 0; kk < D / 16; kk++)
#pragma unroll
    for (int t = 0; t < BN / 32; t++)
      s[t] = mfma_bf16(*reinterpret_cast<const v4i*>(kbase + t * 2 * (32 * D) + kk * 512), qb[kk], s[t]);
}

// ---- Workspace-free form (mxfa_prefill): K arrives as E4M3 codes and is widened in LDS.
// The fp8 codes of the 16 key rows of group g land in the upper half of that group's bf16
// region of the chunk-major tile (g * 32D + 16D .. + 16D), 16-byte chunk (row r, column
// chunk cc) at chunk position 16 cc + r, so that the conversion's reads are contiguous per
// lane; wave g widens group g in place (every code read before its first bf16 store; one
// wave's LDS operations complete in order), so no other wave touches that region.  The K
// scales [BN][D / 32] go to their own small array.
struct P3NSrc {
  __amdgpu_buffer_rsrc_t k8, ks, v, vs;
};

template <int D, bool VBLK = false>
__device__ __forceinline__ void p3n_dma(const P3NSrc& src, uint8_t* kb, uint8_t* ksc, uint8_t* v, int key0, int wave,
                                        int lane, const P3Lane& pl) {
  using L = P3Lds<D>;
  constexpr int KI = 16 * D / 1024;                     // 1 KB instructions per 16-row fp8 group
  const int g = wave;
  const int vk = (lane % 16) * D + (lane / 16) * 16;
#pragma unroll
  for (int m = 0; m < KI; m++)
    dma_lds<16>(src.k8, kb + g * (32 * D) + 16 * D + m * 1024, vk, (key0 + 16 * g) * D + 64 * m);
  // K scales: BN * D / 32 bytes, 256 per dword instruction, from waves 0 (and 1 at D = 256)
  if (wave < (BN * D / 32 + 255) / 256) dma_lds<4>(src.ks, ksc + wave * 256, lane * 4, key0 * (D / 32) + wave * 256);
  // V codes and scales as the workspace form
  if constexpr (VBLK) {
    p3_dma_vblk<D, 4>(src.v, v, key0, wave, lane);
  } else {
    constexpr int VPW = L::VDMA / 4;
    const int i0 = p3_v_instr<D, 4>(wave, 0);
#pragma unroll
    for (int m = 0; m < VPW; m++) {
      const int i = p3_v_instr<D, 4>(wave, m);
      dma_lds<16>(src.v, v + i * 1024, pl.v, key0 * D + (i - i0) * 1024);
    }
  }
#pragma unroll
  for (int m = 0; m < (2 * D + 255) / 256; m++) dma_lds<4>(src.vs, v + L::V + m * 256, pl.s, (key0 / 32) * D + m * 256);
}

// Wave g widens its 16-row group: D / 64 chunks of 16 codes per lane (chunk position lane +
// 64 i: row lane % 16, column chunk cc = lane / 16 + 4 i), exact bf16 (code x 2^(scale -
// 127)), stored as the two bf16 chunks 2 cc and 2 cc + 1 of the row (16 lanes: 256
// contiguous bytes).  Chunk i is read, then stored: its stores cover group bytes [2048 i,
// 2048 i + 2048), below every later read (16 D + 1024 j for j > i, since i < D / 64), so
// one chunk at a time is in registers.
template <int D>
__device__ __forceinline__ void p3n_widen_k(uint8_t* kb, const uint8_t* ksc, int wave, int lane) {
  constexpr int NI = D / 64;
  uint8_t* grp = kb + wave * (32 * D);
  const int rr = lane % 16;
#pragma unroll
  for (int i = 0; i < NI; i++) {
    const int cc = lane / 16 + 4 * i;
    const v4i x = *reinterpret_cast<const v4i*>(grp + 16 * D + 16 * (lane + 64 * i));
    const float f = e8m0_as_float(ksc[(16 * wave + rr) * (D / 32) + cc / 2]);
    *reinterpret_cast<v4i*>(grp + 256 * (2 * cc) + 16 * rr) = fp8x8_to_bf16x8((uint32_t)x[0], (uint32_t)x[1], f);
    *reinterpret_cast<v4i*>(grp + 256 * (2 * cc + 1) + 16 * rr) = fp8x8_to_bf16x8((uint32_t)x[2], (uint32_t)x[3], f);
  }
}

// E3M2 V codes (low 6 bits) -> E5M2 codes of the same bits moved (sign 5 -> 7): an E5M2 byte
// with exponent field e3 and mantissa m2 is the E3M2 value x 2^-12, subnormals included
// (2^-14 x 0.m vs 2^-2 x 0.m), so the PV MFMA reads V as E5M2 and O is scaled by 2^12 at the
// end (exact).  The tile's BN x D bytes, 16 per thread and pass, rewritten in place.
template <int D>
__device__ __forceinline__ void p3n_v_e3m2_to_e5m2(uint8_t* v, int tid) {
  constexpr int NI = BN * D / 16 / 256;
#pragma unroll
  for (int i = 0; i < NI; i++) {
    v4i* ptr = reinterpret_cast<v4i*>(v + 16 * (tid + 256 * i));
    v4i w = *ptr;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const uint32_t u = (uint32_t)w[e];
      w[e] = (int)((u & 0x1f1f1f1fu) | ((u & 0x20202020u) << 2));
    }
    *ptr = w;
  }
}

// The lane index, recomputed where it is used (two VALU instructions the compiler cannot
// merge with an earlier copy): addresses derived from it need no register across the loop.
__device__ __forceinline__ int fresh_lane() {
  int l;
  __asm__ volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}

// NOWS: the workspace-free form (mxfa_prefill): K read as E4M3 codes and widened to bf16 in
// LDS by p3n_widen_k at the top of every block (one K stage), V read from the caller's array;
// VE3: V is E3M2, rewritten in LDS as E5M2 (p3n_v_e3m2_to_e5m2), O scaled by 2^12.
// VBLK: V is E3M2 in the block-packed layout ([Skc / 32][D][24 bytes] per (b, KV head)),
// copied into LDS as it is and read by the PV MFMA as its fp6 operand (pv_parts_blk).
template <int D, bool SOFTCAP, int PR, bool TRACE = false, bool NOWS = false, bool VE3 = false, bool VBLK = false>
__device__ void prefill3_impl(const FaArgs& a) {
  using L = P3Lds<D>;
  constexpr int NW = P3Waves<D>::N;
  fp32_flush_denormals();   // pipe_softmax's R1 flush
  constexpr bool K1 = NOWS || p3_one_k_stage<D>();
  __shared__ __attribute__((aligned(16))) uint8_t sKb0[L::KB];
  __shared__ __attribute__((aligned(16))) uint8_t sKb1[K1 ? 16 : L::KB];
  __shared__ __attribute__((aligned(16))) uint8_t sKs[NOWS ? (BN * D / 32 > 256 ? BN * D / 32 : 256) : 16];
  __shared__ __attribute__((aligned(256))) uint8_t sV0[L::V + L::SCB];   // 256-aligned: pv_parts' addresses
  __shared__ __attribute__((aligned(256))) uint8_t sV1[L::V + L::SCB];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 31, h = lane >> 5;
  const int nwg = (int)(gridDim.x * gridDim.y);
  const int lin = (int)(blockIdx.y * gridDim.x + blockIdx.x);
  const int xcd = lin & 7, per = nwg >> 3, rem = nwg & 7;
  const int start_x = xcd * per + min(xcd, rem), cnt_x = per + (xcd < rem ? 1 : 0);
  const int li = lin >> 3;
  const int nh_x = cnt_x / a.n_qblk;
  const bool whole_heads = start_x % a.n_qblk == 0 && cnt_x % a.n_qblk == 0;
  const int item = start_x + (whole_heads ? (li % nh_x) * a.n_qblk + li / nh_x : li);
  const int qx = TRACE ? a.tr_qx : item % a.n_qblk, qy = TRACE ? a.tr_qy : item / a.n_qblk;
  const int qblk = a.causal ? (a.n_qblk - 1 - qx) : qx;
  const int chunks = a.group / a.hpw;
  const int bk = qy / chunks;
  const int hc = qy % chunks;
  const int b = bk / a.Hkv, kvh = bk % a.Hkv;
  const int head = kvh * a.group + hc * a.hpw + (wave % a.hpw);
  const int q0 = qblk * a.qpw;
  const int qw0 = q0 + (wave / a.hpw) * 32;
  const int qi = qw0 + r;
  const bool qvalid = qi < a.Sq;
  const int qpos = a.q_pos0 + qi;
  const bool traced = TRACE && head == a.tr_head && qw0 == a.tr_q0;   // wave-uniform

  const int64_t bh = (int64_t)b * a.Hq + head;
  v4i qb[D / 16];
  load_q<D>(qb, a.q + (bh * a.Sq + qi) * D, a.qs + (bh * a.Sq + qi) * (D / 32), qvalid, h);

  const int qmax_wg = min(q0 + a.qpw, a.Sq) - 1;
  const int nkb = (a.Sk + BN - 1) / BN;
  int j0 = 0, j1 = nkb;
  if (a.window > 0) j0 = max(0, a.q_pos0 + q0 - a.window + 1) / BN;
  if (a.causal) j1 = min(nkb, max(0, a.q_pos0 + qmax_wg) / BN + 1);
  const int wq_lo = a.q_pos0 + qw0, wq_hi = a.q_pos0 + min(qw0 + 31, a.Sq - 1);
  const bool wave_live = qw0 < a.Sq;

  // V codes: the caller's E4M3 V, or its E4M3 copy (dense, Sk keys) when V is E3M2
  const P3Src src = NOWS   ? P3Src{}
                    : VBLK ? P3Src{buf_rsrc(a.kbf, (int64_t)bk * a.Sk * (2 * D), (int64_t)a.Sk * (2 * D)),
                                   buf_rsrc(a.v, (int64_t)bk * (a.Skc / 32) * (24 * D), (int64_t)(a.Sk / 32) * (24 * D)),
                                   buf_rsrc(a.vs, (int64_t)bk * (a.Skc / 32) * D, (int64_t)(a.Sk / 32) * D)}
                           : p3_src(a.kbf + (int64_t)bk * a.Sk * (2 * D),
                                    a.vws ? a.vws + (int64_t)bk * a.Sk * D : a.v + (int64_t)bk * a.Skc * D,
                                    a.vs + (int64_t)bk * (a.Skc / 32) * D, a.Sk, D);
  // workspace-free: the caller's K codes and scales, V and V scales (Skc keys apart), each
  // resource ending at key Sk
  const P3NSrc nsrc = !NOWS ? P3NSrc{}
                            : P3NSrc{buf_rsrc(a.k, (int64_t)bk * a.Skc * D, (int64_t)a.Sk * D),
                                     buf_rsrc(a.ks, (int64_t)bk * a.Skc * (D / 32), (int64_t)a.Sk * (D / 32)),
                                     VBLK ? buf_rsrc(a.v, (int64_t)bk * (a.Skc / 32) * (24 * D), (int64_t)(a.Sk / 32) * (24 * D))
                                          : buf_rsrc(a.v, (int64_t)bk * a.Skc * D, (int64_t)a.Sk * D),
                                     buf_rsrc(a.vs, (int64_t)bk * (a.Skc / 32) * D, (int64_t)(a.Sk / 32) * D)};
  const P3Lane pl = p3_lane<D, NW>(wave, lane);
  // loop-invariant operands in VGPRs at three waves per SIMD (D <= 128), in SGPRs at two (D =
  // 256: there an SGPR operand issues at the full-rate op's speed and saves the register)
  const float c = SOFTCAP ? 1.0f : (D <= 128 ? in_vgpr(a.c_log2) : a.c_log2);

  v16f o[D / 32];
#pragma unroll
  for (int dt = 0; dt < D / 32; dt++) o[dt] = (v16f){};
  float m = -INFINITY, l = 0.0f;

  // the wave's rows end at or past Sq (or it has none): every block is masked
  const bool edge_wave = __builtin_amdgcn_readfirstlane((qw0 + 31 >= a.Sq) || !wave_live);
  auto need_mask = [&](int j) {
    const int key0 = j * BN, key1 = key0 + BN - 1;
    return edge_wave || (bool)__builtin_amdgcn_readfirstlane((key1 >= a.Sk) || (a.causal && key1 > wq_lo) ||
                                                              (a.window > 0 && key0 + a.window <= wq_hi));
  };

  if (j0 < j1) {
    if constexpr (NOWS) p3n_dma<D, VBLK>(nsrc, sKb0, sKs, sV0, j0 * BN, wave, lane, pl);
    else p3_dma<D, NW, true, true, VBLK>(src, sKb0, sV0, j0 * BN, wave, pl, lane);
  }
  __builtin_amdgcn_s_waitcnt(0x0070 | 0x0f00 | 0);   // vmcnt(0)
  __syncthreads();

  auto step = [&](auto stc, int j) {
    constexpr int ST = decltype(stc)::value;
    uint8_t* kb_cur = K1 || !ST ? sKb0 : sKb1;
    uint8_t* kb_dma = K1 || ST ? sKb0 : sKb1;
    uint8_t* v_cur = ST ? sV1 : sV0;
    uint8_t* v_dma = ST ? sV0 : sV1;
    // the DMA instructions of block j+1 (also past the last block: keys >= Sk read 0, and
    // nothing reads that stage) are issued between the score MFMAs of block j, or -- one K
    // stage -- once every wave has read K(j), while the MFMAs run
    v16f sc[BN / 32];
    if constexpr (NOWS) {
      // widen this block's K group of the wave (and rewrite an E3M2 V tile as E5M2), then
      // let every wave see the whole tile
      // (lane ids recomputed here: addresses held across the loop would not fit at D = 256)
      p3n_widen_k<D>(sKb0, sKs, wave, fresh_lane());
      if constexpr (VE3) p3n_v_e3m2_to_e5m2<D>(v_cur, 64 * wave + fresh_lane());
      __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0)
      __builtin_amdgcn_s_barrier();
    }
    // D <= 128: the score MFMAs at raised wave priority, so that the SIMD's arbiter issues them
    // ahead of the other two workgroups' softmax VALU (about 1% faster on the S = 4096 GQA
    // prefill); D = 256 (two waves per SIMD) runs about 0.5% faster without it
    if constexpr (D <= 128) __builtin_amdgcn_s_setprio(1);
    // the score-operand address from the lane id held across the loop (one register; about
    // 1% faster on the S = 4096 GQA prefill than recomputing it per block); the softcap
    // kernels, one register short, recompute it
    p3_qk<D>(sc, qb, kb_cur, SOFTCAP ? fresh_lane() : lane);
    if constexpr (K1) {
      __builtin_amdgcn_s_waitcnt(0xc07f);   // lgkmcnt(0): this wave's K operand reads are done
      __builtin_amdgcn_s_barrier();
      if constexpr (NOWS) p3n_dma<D, VBLK>(nsrc, kb_dma, sKs, v_dma, (j + 1) * BN, wave, fresh_lane(), pl);
      else p3_dma<D, NW, true, true, VBLK>(src, kb_dma, v_dma, (j + 1) * BN, wave, pl, fresh_lane());
    } else {
      p3_dma<D, NW, true, true, VBLK>(src, kb_dma, v_dma, (j + 1) * BN, wave, pl, lane);
      p3_dma_interleave<D>();
    }
    if constexpr (D <= 128) __builtin_amdgcn_s_setprio(0);
    pipe_scores<SOFTCAP, D <= 128>(sc, a);
    if (need_mask(j)) {
      const int ln = fresh_lane();
      int klo, khi;
      key_limits(a, a.q_pos0 + qw0 + (ln & 31), qw0 + (ln & 31) < a.Sq, klo, khi);
      pipe_mask<SOFTCAP>(sc, j * BN, klo, khi, ln >> 5);
    }
    if constexpr (TRACE) {
      if (traced) {
#pragma unroll
        for (int t = 0; t < BN / 32; t++)
#pragma unroll
          for (int i = 0; i < 16; i++) {
            const int key = j * BN + 32 * t + 8 * (i >> 2) + 4 * h + (i & 3);
            if (key < a.Sk) a.tr_s[(int64_t)r * a.Sk + key] = SOFTCAP ? capped_score(sc[t][i], a) : sc[t][i];
          }
      }
    }
    v8i pb;
    int psc[BN / 32];
    float corr;
    pipe_softmax<SOFTCAP, PR, D <= 128>(m, l, sc, pb, psc, corr, c, -2.0f * a.cap_log2, a.cap_log2);
    if constexpr (TRACE) {
      const float lrow = pair_sum(l);
      if (traced) {
#pragma unroll
        for (int t = 0; t < BN / 32; t++) {
#pragma unroll
          for (int g = 0; g < 4; g++)
#pragma unroll
            for (int bb = 0; bb < 4; bb++) {
              const int key = j * BN + 32 * t + 8 * g + 4 * h + bb;
              if (key < a.Sk) a.tr_p[(int64_t)r * a.Sk + key] = (uint8_t)((uint32_t)pb[4 * t + g] >> (8 * bb));
            }
          if (h == 0 && j * BN + 32 * t < a.Sk) a.tr_ps[(int64_t)r * (a.Sk / 32) + (j * BN) / 32 + t] = (uint8_t)psc[t];
        }
        if (h == 0) {
          a.tr_ml[((int64_t)j * 32 + r) * 2] = m;
          a.tr_ml[((int64_t)j * 32 + r) * 2 + 1] = lrow;
        }
      }
    }
    if (__any(corr != 1.0f)) {
#pragma unroll
      for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
        for (int i = 0; i < 16; i++) o[dt][i] *= corr;
    }
    // D <= 128: the PV addresses stay in registers (loop-invariant); D = 256 has no room
    if constexpr (VBLK) pv_parts_blk<D, D == 256 ? 2 : 1>(o, v_cur, pb, psc, D == 256 ? fresh_lane() : lane);
    else pv_parts<D, D == 256 ? 2 : 1, VE3>(o, v_cur, pb, psc, D == 256 ? fresh_lane() : lane);
    __builtin_amdgcn_s_waitcnt(0x0070 | 0x0000 | 0);   // vmcnt(0) lgkmcnt(0): next stage landed
    __builtin_amdgcn_s_barrier();
  };
  for (int j = j0; j < j1; j += 2) {
    step(std::integral_constant<int, 0>{}, j);
    if (j + 1 < j1) step(std::integral_constant<int, 1>{}, j + 1);
  }

  const float lt = pair_sum(l);
  // (an E3M2 V read as E5M2 carries 2^-12: undone here, exactly)
  const float inv = lt > 0.0f ? (VE3 ? 4096.0f : 1.0f) / lt : 0.0f;
  if constexpr (D >= 128 && !TRACE) {
    // O through LDS (store_o_lds), in a private 8 KB slice of the K tiles (one K stage at D =
    // 128: the V tiles for waves 2 and 3), free after the loop's last barrier (96 -> 68 MB
    // fetched and 161 -> 134 MB written on the S = 4096 GQA prefill)
    float* const ldsw = reinterpret_cast<float*>(
        D == 256 ? sKb0 + wave * 8192
        : K1     ? (wave < 2 ? sKb0 + wave * 8192 : wave == 2 ? sV0 : sV1)
                 : (wave < 2 ? sKb0 : sKb1) + (wave & 1) * 8192);
    store_o_lds<D>(o, inv, ldsw, a.o + bh * a.Sq * D, qw0, a.Sq, lane);
  } else if (qvalid) {
    float* orow = a.o + (bh * a.Sq + qi) * D;
#pragma unroll
    for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const float4 w = make_float4(o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv, o[dt][4 * g + 2] * inv,
                                     o[dt][4 * g + 3] * inv);
        *reinterpret_cast<float4*>(orow + dt * 32 + 8 * g + 4 * h) = w;
      }
  }
}

#define MXFA_PREFILL3(D, SC, PR, NAME)                                                           \
  extern "C" __global__ void __launch_bounds__(64 * P3Waves<D>::N, p3_one_k_stage<D>() ? 2 : 3) NAME(FaArgs a) { \
    prefill3_impl<D, SC, PR>(a);                                                                    \
  }
MXFA_PREFILL3(64, false, P_R1, mxfa_prefill3_d64)
MXFA_PREFILL3(128, false, P_R1, mxfa_prefill3_d128)
MXFA_PREFILL3(64, true, P_R1, mxfa_prefill3_d64_softcap)
MXFA_PREFILL3(128, true, P_R1, mxfa_prefill3_d128_softcap)
MXFA_PREFILL3(64, false, P_R2, mxfa_prefill3_d64_r2)
MXFA_PREFILL3(128, false, P_R2, mxfa_prefill3_d128_r2)
MXFA_PREFILL3(64, true, P_R2, mxfa_prefill3_d64_softcap_r2)
MXFA_PREFILL3(128, true, P_R2, mxfa_prefill3_d128_softcap_r2)
MXFA_PREFILL3(256, false, P_R1, mxfa_prefill3_d256)
MXFA_PREFILL3(256, true, P_R1, mxfa_prefill3_d256_softcap)
MXFA_PREFILL3(256, false, P_R2, mxfa_prefill3_d256_r2)
MXFA_PREFILL3(256, true, P_R2, mxfa_prefill3_d256_softcap_r2)
// E3M2 V in the block-packed layout (the pre-pass widens K only)
#define MXFA_PREFILL3B(D, SC, PR, NOWS, NAME)                                                        \
  extern "C" __global__ void __launch_bounds__(256, D == 256 ? 2 : 3) NAME(FaArgs a) {               \
    prefill3_impl<D, SC, PR, false, NOWS, false, true>(a);                                           \
  }
#define MXFA_PREFILL3B_ALL(D)                                                                        \
  MXFA_PREFILL3B(D, false, P_R1, false, mxfa_prefill3_d##D##_blk)                                    \
  MXFA_PREFILL3B(D, true, P_R1, false, mxfa_prefill3_d##D##_softcap_blk)                             \
  MXFA_PREFILL3B(D, false, P_R2, false, mxfa_prefill3_d##D##_r2_blk)                                 \
  MXFA_PREFILL3B(D, true, P_R2, false, mxfa_prefill3_d##D##_softcap_r2_blk)                          \
  MXFA_PREFILL3B(D, false, P_R1, true, mxfa_prefill3n_d##D##_blk)                                    \
  MXFA_PREFILL3B(D, true, P_R1, true, mxfa_prefill3n_d##D##_softcap_blk)                             \
  MXFA_PREFILL3B(D, false, P_R2, true, mxfa_prefill3n_d##D##_r2_blk)                                 \
  MXFA_PREFILL3B(D, true, P_R2, true, mxfa_prefill3n_d##D##_softcap_r2_blk)
MXFA_PREFILL3B_ALL(64)
MXFA_PREFILL3B_ALL(128)
MXFA_PREFILL3B_ALL(256)

// Workspace-free prefill (mxfa_prefill, and mxfa_prefill_ws where widening K per workgroup
// costs less than the pre-pass): K widened in LDS, E3M2 V read as E5M2.
#define MXFA_PREFILL3N(D, SC, PR, VE3, NAME)                                                        \
  extern "C" __global__ void __launch_bounds__(256, D == 256 ? 2 : 3) NAME(FaArgs a) {               \
    prefill3_impl<D, SC, PR, false, true, VE3>(a);                                                   \
  }
MXFA_PREFILL3N(64, false, P_R1, false, mxfa_prefill3n_d64)
MXFA_PREFILL3N(128, false, P_R1, false, mxfa_prefill3n_d128)
MXFA_PREFILL3N(256, false, P_R1, false, mxfa_prefill3n_d256)
MXFA_PREFILL3N(64, true, P_R1, false, mxfa_prefill3n_d64_softcap)
MXFA_PREFILL3N(128, true, P_R1, false, mxfa_prefill3n_d128_softcap)
MXFA_PREFILL3N(256, true, P_R1, false, mxfa_prefill3n_d256_softcap)
MXFA_PREFILL3N(64, false, P_R2, false, mxfa_prefill3n_d64_r2)
MXFA_PREFILL3N(128, false, P_R2, false, mxfa_prefill3n_d128_r2)
MXFA_PREFILL3N(256, false, P_R2, false, mxfa_prefill3n_d256_r2)
MXFA_PREFILL3N(64, true, P_R2, false, mxfa_prefill3n_d64_softcap_r2)
MXFA_PREFILL3N(128, true, P_R2, false, mxfa_prefill3n_d128_softcap_r2)
MXFA_PREFILL3N(256, true, P_R2, false, mxfa_prefill3n_d256_softcap_r2)
MXFA_PREFILL3N(64, false, P_R1, true, mxfa_prefill3n_d64_e3m2)
MXFA_PREFILL3N(128, false, P_R1, true, mxfa_prefill3n_d128_e3m2)
MXFA_PREFILL3N(256, false, P_R1, true, mxfa_prefill3n_d256_e3m2)
MXFA_PREFILL3N(64, true, P_R1, true, mxfa_prefill3n_d64_softcap_e3m2)
MXFA_PREFILL3N(128, true, P_R1, true, mxfa_prefill3n_d128_softcap_e3m2)
MXFA_PREFILL3N(256, true, P_R1, true, mxfa_prefill3n_d256_softcap_e3m2)
MXFA_PREFILL3N(64, false, P_R2, true, mxfa_prefill3n_d64_r2_e3m2)
MXFA_PREFILL3N(128, false, P_R2, true, mxfa_prefill3n_d128_r2_e3m2)
MXFA_PREFILL3N(256, false, P_R2, true, mxfa_prefill3n_d256_r2_e3m2)
MXFA_PREFILL3N(64, true, P_R2, true, mxfa_prefill3n_d64_softcap_r2_e3m2)
MXFA_PREFILL3N(128, true, P_R2, true, mxfa_prefill3n_d128_softcap_r2_e3m2)
MXFA_PREFILL3N(256, true, P_R2, true, mxfa_prefill3n_d256_softcap_r2_e3m2)

// Stage trace of the same kernel (one workgroup; mxfa_prefill_trace).
#define MXFA_PREFILL3_TRACE(D, SC, PR, NAME)                                                                  \
  extern "C" __global__ void __launch_bounds__(64 * P3Waves<D>::N, 1) NAME(FaArgs a) {                        \
    prefill3_impl<D, SC, PR, true>(a);                                                                        \
  }
MXFA_PREFILL3_TRACE(64, false, P_R1, mxfa_prefill3_trace_d64)
MXFA_PREFILL3_TRACE(128, false, P_R1, mxfa_prefill3_trace_d128)
MXFA_PREFILL3_TRACE(256, false, P_R1, mxfa_prefill3_trace_d256)
MXFA_PREFILL3_TRACE(64, true, P_R1, mxfa_prefill3_trace_d64_softcap)
MXFA_PREFILL3_TRACE(128, true, P_R1, mxfa_prefill3_trace_d128_softcap)
MXFA_PREFILL3_TRACE(256, true, P_R1, mxfa_prefill3_trace_d256_softcap)
MXFA_PREFILL3_TRACE(64, false, P_R2, mxfa_prefill3_trace_d64_r2)
MXFA_PREFILL3_TRACE(128, false, P_R2, mxfa_prefill3_trace_d128_r2)
MXFA_PREFILL3_TRACE(256, false, P_R2, mxfa_prefill3_trace_d256_r2)
MXFA_PREFILL3_TRACE(64, true, P_R2, mxfa_prefill3_trace_d64_softcap_r2)
MXFA_PREFILL3_TRACE(128, true, P_R2, mxfa_prefill3_trace_d128_softcap_r2)
MXFA_PREFILL3_TRACE(256, true, P_R2, mxfa_prefill3_trace_d256_softcap_r2)

// ---------------------------------------------------------------------------
// Decode (q_len = 1, split-KV).  The 64-key blocks of each (b, KV head) are dealt to
// nparts interleaved partials (partial i: blocks i, i + nparts, ...); one wave runs each
// partial as an independent streaming pass and produces its (m, l, O); the partials are
// merged in part order (inside the workgroup, or by mxfa_decode_combine).  The group's
// query heads are the wave's query columns (column c = head kvh*group + c).
// ---------------------------------------------------------------------------
// One wave per partial of one (b, KV head); its 32 score columns are the group's query
// heads (columns >= group are padding).
// K and V are read in block order (whole lines per load instruction, non-temporal) and
// pass through the wave's LDS slot in turn: K is read back in the split-d mapping and
// dequantized to bf16 right before each score MFMA, then V takes the slot for the
// ds_read_b64_tr_b8 reads of the PV step.  Small per-wave LDS and register footprints
// give two workgroups per CU at D <= 128, whose waves hide each other's load latency; at
// D = 256 one workgroup per CU keeps twice the bytes per wave in flight.
// ---------------------------------------------------------------------------
template <int D, bool SOFTCAP, int PR, bool VBLK = false>
__device__ void decode_split_impl(const FaArgs& a) {
  constexpr int NW = 4;
  constexpr int NT = BN / 32;
  constexpr int CPR = D / 16;                         // 16-byte chunks per V row
  constexpr int PERW = BN * CPR / 64;                 // K (and E4M3 V) chunks per lane
  constexpr int PERWV = VBLK ? 3 * D / 64 : PERW;     // V chunks per lane (block-packed: 48 D bytes)
  constexpr int SCW = BN * D / 32 / 4;                // V scale dwords per block
  constexpr int SCPL = (SCW + 63) / 64;               // V scale dwords per lane
  constexpr int KC = D / 32;                          // 16-byte K chunks per lane per tile
  constexpr int KSB = D / 64;                         // K scale bytes per half-row
  constexpr int KP = Lds<D>::KP;
  __shared__ __attribute__((aligned(16))) uint8_t sV[NW][Lds<D>::TILE];
  __shared__ __attribute__((aligned(16))) uint8_t sVs[NW][Lds<D>::SC];
  // D = 256: the bf16 Q operand (64 registers) waits in LDS, MFMA kk's 64 lanes in one
  // contiguous 1 KB row, so that a block's K and V codes stay in flight in registers
  constexpr bool QLDS = D == 256;
  __shared__ __attribute__((aligned(16))) v4i sQ[QLDS ? NW : 1][QLDS ? D / 16 * 64 : 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 31, h = lane >> 5;
  // one (batch, KV head, chunk) item per wave, items numbered chunk-fastest over the
  // whole grid: every wave of a workgroup has work (the waves share nothing)
  // Waves past the last item have no work; they stay for the workgroup barrier of the
  // fused merge below (their loads use the last item's addresses and read nothing).
  const int n_items = a.B * a.Hkv * a.n_qblk;
  const int item = blockIdx.x * NW + wave;
  const bool active = item < n_items;
  if (!active && !a.fuse_combine) return;
  const int it = active ? item : n_items - 1;
  const int bk = it / a.n_qblk, part = it - bk * a.n_qblk;
  const int b = bk / a.Hkv, kvh = bk % a.Hkv;
  const bool qvalid = r < a.group;
  const int head = kvh * a.group + (qvalid ? r : 0);
  const int64_t bh = (int64_t)b * a.Hq + head;
  const int qpos = a.q_pos0;                          // the single query's position

  v4i qb[QLDS ? 1 : D / 16];
  if constexpr (QLDS) {
    v4i qt[D / 16];
    load_q_split<D>(qt, a.q + bh * D, a.qs + bh * (D / 32), qvalid, h);
#pragma unroll
    for (int kk = 0; kk < D / 16; kk++) sQ[wave][kk * 64 + lane] = qt[kk];
  } else {
    load_q_split<D>(qb, a.q + bh * D, a.qs + bh * (D / 32), qvalid, h);
  }

  // buffer resources end at Sk: rows past it read 0
  const __amdgpu_buffer_rsrc_t rk = buf_rsrc(a.k, (int64_t)bk * a.Skc * D, (int64_t)a.Sk * D);
  const __amdgpu_buffer_rsrc_t rks = buf_rsrc(a.ks, (int64_t)bk * a.Skc * (D / 32), (int64_t)a.Sk * (D / 32));
  const __amdgpu_buffer_rsrc_t rv =
      VBLK ? buf_rsrc(a.v, (int64_t)bk * (a.Skc / 32) * (24 * D), (int64_t)(a.Sk / 32) * (24 * D))
           : buf_rsrc(a.v, (int64_t)bk * a.Skc * D, (int64_t)a.Sk * D);
  const __amdgpu_buffer_rsrc_t rvs = buf_rsrc(a.vs, (int64_t)bk * (a.Skc / 32) * D, (int64_t)(a.Sk / 32) * D);

  int klo, khi;
  key_limits(a, qpos, qvalid, klo, khi);
  // Partial `part` of n_qblk takes the key blocks part, part + n_qblk, ... (interleaved:
  // the partial waves of a head, which share a workgroup, read adjacent blocks at the
  // same time).  The visible range of the (single) query position is uniform over the
  // wave: blocks outside it contribute nothing (P = 0, the max unchanged) and are not
  // visited; blocks inside it need no mask.  Padding columns (r >= group, Q = 0) are not
  // masked: their scores are 0, their state stays finite and is never written.
  int klo_u, khi_u;
  key_limits(a, qpos, true, klo_u, khi_u);
  const int kstride = a.n_qblk * BN;
  const int blo = klo_u / BN;                         // first visible block
  const int bfirst = blo <= part ? part : part + (blo - part + a.n_qblk - 1) / a.n_qblk * a.n_qblk;
  const int kfirst = bfirst * BN, klast = active ? khi_u + 1 : kfirst;

  WaveState<D> st;
#pragma unroll
  for (int dt = 0; dt < D / 32; dt++) st.o[dt] = (v16f){};
  st.m = -INFINITY;
  st.l = 0.0f;

  // K and V codes are read once per call, whole 128-byte lines per instruction (16 bytes
  // per lane, consecutive lanes on consecutive bytes of a block), with non-temporal loads
  // (cache policy nt): measured on c5, 11% faster per operand than the default policy.
  // Loads in the split-d mapping itself (a lane reading half a key row) cover 32 bytes of
  // each line per instruction, and nt on those costs 18%.
  constexpr int kNonTemporal = 2;
  // K codes of a block in block order (moved to the split-d mapping through the wave's
  // LDS slot before the scores) and the E8M0 scales of this lane's K half-rows (keys
  // key0 + 32t + r).  A disabled load gets an offset past every resource: it reads nothing
  // and returns 0; no branch, so the waits on the other loads stay partial.
  // KH: the block's K loads go out in KH parts (part u: tiles NT/KH u ..), each just before
  // the scores that free its registers' previous contents -- at D = 256 the second tile's
  // loads wait for the first tile's scores, which keeps the peak register demand in bounds
  constexpr int KH = QLDS ? 2 : 1;
  v4i kr[PERW];
  uint32_t ksr[NT];
  auto load_k = [&](int key0, bool on, int u) {
#pragma unroll
    for (int i = u * (PERW / KH); i < (u + 1) * (PERW / KH); i++) {
      const int c = lane + 64 * i;
      const uint32_t ko = on ? (uint32_t)((key0 + c / CPR) * D + (c % CPR) * 16) : 0x80000000u;
      kr[i] = __builtin_amdgcn_raw_buffer_load_b128(rk, ko, 0, kNonTemporal);
    }
#pragma unroll
    for (int t = u * (NT / KH); t < (u + 1) * (NT / KH); t++) {
      const int row = key0 + 32 * t + r;
      const uint32_t so = on ? (uint32_t)(row * (D / 32) + KSB * h) : 0x80000000u;
      if constexpr (KSB == 4)
        ksr[t] = __builtin_amdgcn_raw_buffer_load_b32(rks, so, 0, 0);
      else if constexpr (KSB == 2)
        ksr[t] = __builtin_amdgcn_raw_buffer_load_b16(rks, so, 0, 0);
      else
        ksr[t] = __builtin_amdgcn_raw_buffer_load_b8(rks, so, 0, 0);
    }
  };
  // V codes and scales of a block (stored to the wave's LDS slot after its scores); block-
  // packed V: the block's 48 D contiguous bytes, chunk c at byte 16 c of the slot
  v4i vr[PERWV];
  uint32_t vsr[SCPL];
  auto load_v = [&](int key0, bool on) {
#pragma unroll
    for (int i = 0; i < PERWV; i++) {
      const int c = lane + 64 * i;
      const uint32_t vo = !on ? 0x80000000u
                          : VBLK ? (uint32_t)((key0 / 32) * (24 * D) + 16 * c)
                                 : (uint32_t)((key0 + c / CPR) * D + (c % CPR) * 16);
      vr[i] = __builtin_amdgcn_raw_buffer_load_b128(rv, vo, 0, kNonTemporal);
    }
#pragma unroll
    for (int i = 0; i < SCPL; i++) {
      const int d = lane + 64 * i;
      const uint32_t so = on && d < SCW ? (uint32_t)((key0 / 32) * D + 4 * d) : 0x80000000u;
      vsr[i] = __builtin_amdgcn_raw_buffer_load_b32(rvs, so, 0, kNonTemporal);
    }
  };
  // one block ahead: K(j+1) goes out once K(j) is in LDS, V(j+1) once V(j) is, and both
  // stay in flight through the scores, softmax and PV of block j
#pragma unroll
  for (int u = 0; u < KH; u++) load_k(kfirst, kfirst < klast, u);
  load_v(kfirst, kfirst < klast);
  for (int key0 = kfirst; key0 < klast; key0 += kstride) {
    // K tile into the wave's slot (row pitch KP, like V), then each lane reads back its
    // half-rows.  LDS operations of one wave complete in order, so the reads see the
    // tile; the compiler barriers keep this block's K writes after the previous block's
    // PV reads and the V writes below after these K reads (the same bytes, other lanes).
    __asm__ volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < PERW; i++) {
      const int c = lane + 64 * i;
      *reinterpret_cast<v4i*>(&sV[wave][(c / CPR) * KP + (c % CPR) * 16]) = kr[i];
    }
    // the next block's K goes out once this block's codes are in LDS (at D = 256 half of it
    // waits for the first tile's scores); its scales replace this block's, which the
    // scores still need: they are kept in ksc
    uint32_t ksc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) ksc[t] = ksr[t];
    // scores: K dequantized to bf16 just before each MFMA
    v16f sc[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
      if (t % (NT / KH) == 0) load_k(key0 + kstride, key0 + kstride < klast, t / (NT / KH));
      // K half-row chunks read from LDS KR at a time (D = 256: half the row per read group)
      constexpr int KR = QLDS ? KC / 2 : KC;
      sc[t] = (v16f){};
#pragma unroll
      for (int c0 = 0; c0 < KC; c0 += KR) {
        v4i kt[KR];
#pragma unroll
        for (int c = 0; c < KR; c++)
          kt[c] = *reinterpret_cast<const v4i*>(&sV[wave][(32 * t + r) * KP + h * (D / 2) + 16 * (c0 + c)]);
#pragma unroll
        for (int k2 = 0; k2 < 2 * KR; k2++) {
          const int kk = 2 * c0 + k2;
          const v4i& w = kt[k2 / 2];
          const float scale = e8m0_as_float((ksc[t] >> (8 * (kk / 4))) & 0xffu);
          const v4i ka = fp8x8_to_bf16x8((uint32_t)w[2 * (kk & 1)], (uint32_t)w[2 * (kk & 1) + 1], scale);
          sc[t] = mfma_bf16(ka, QLDS ? sQ[wave][kk * 64 + lane] : qb[kk], sc[t]);
        }
      }
    }
    __asm__ volatile("" ::: "memory");
#pragma unroll
    for (int i = 0; i < PERWV; i++) {
      const int c = lane + 64 * i;
      v4i zv = vr[i];
      if (!VBLK && a.v_e3m2) {
#pragma unroll
        for (int w = 0; w < 4; w++) zv[w] = (int)e3m2x4_to_e4m3x4((uint32_t)zv[w]);
      }
      *reinterpret_cast<v4i*>(&sV[wave][VBLK ? 16 * c : (c / CPR) * KP + (c % CPR) * 16]) = zv;
    }
#pragma unroll
    for (int i = 0; i < SCPL; i++)
      if (lane + 64 * i < SCW) *reinterpret_cast<uint32_t*>(&sVs[wave][4 * (lane + 64 * i)]) = vsr[i];
    load_v(key0 + kstride, key0 + kstride < klast);
    // LDS operations of one wave complete in order: the V tile written above is in place
    // for the transposed reads, and the next block's writes follow this block's reads
    const bool mask = key0 < klo_u || key0 + BN - 1 > khi_u;
    softmax_pv<D, SOFTCAP, PR, VBLK>(st, sc, sV[wave], sVs[wave], key0, klo, khi, mask, a, lane);
  }

  float l = pair_sum(st.l);
  const int nparts = a.n_qblk;
  if (a.fuse_combine) {
    // All chunks of a (b, KV head) are waves of this workgroup (nparts divides NW, group
    // <= 16).  Every wave leaves (O, m, l) of its valid columns in its own (now unused)
    // LDS slot; then all threads merge: each takes 4 consecutive d of one query head and
    // combines the chunks in chunk order with the formula of mxfa_decode_combine.
    const int G = a.group;
    float* po = reinterpret_cast<float*>(sV[wave]);
    float* pml = reinterpret_cast<float*>(sVs[wave]);
    // slot layout: float4 (dt, g) of column (h, r) at [(dt * 4 + g) * 2G + h G + r]
    if (active && qvalid) {
#pragma unroll
      for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
        for (int g = 0; g < 4; g++)
          reinterpret_cast<float4*>(po)[(dt * 4 + g) * 2 * G + h * G + r] =
              make_float4(st.o[dt][4 * g], st.o[dt][4 * g + 1], st.o[dt][4 * g + 2], st.o[dt][4 * g + 3]);
      if (h == 0) {
        pml[2 * r] = st.m;
        pml[2 * r + 1] = l;
      }
    }
    __syncthreads();
    const float c = SOFTCAP ? 1.0f : a.c_log2;
    const int heads_wg = NW / nparts, per_head = G * (D / 4);
    for (int u = tid; u < heads_wg * per_head; u += 64 * NW) {
      const int hg = u / per_head, rem = u - hg * per_head;
      const int q = rem / (D / 4), d = 4 * (rem - q * (D / 4));
      const int item0 = blockIdx.x * NW + hg * nparts;
      if (item0 >= n_items) break;
      const int bk0 = item0 / nparts;
      // register position of d: dt = d / 32, g = (d % 32) / 8, half = (d % 8) / 4
      const int fi = ((d >> 5) * 4 + ((d & 31) >> 3)) * 2 * G + ((d & 7) >> 2) * G + q;
      float M = -INFINITY;
      for (int i = 0; i < nparts; i++) {
        const float* qml = reinterpret_cast<const float*>(sVs[hg * nparts + i]);
        if (qml[2 * q + 1] > 0.0f) M = fmaxf(M, qml[2 * q]);
      }
      float L = 0.0f;
      float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (M != -INFINITY) {
        const float mc = M * c;
        for (int i = 0; i < nparts; i++) {
          const float* qml = reinterpret_cast<const float*>(sVs[hg * nparts + i]);
          const float li = qml[2 * q + 1];
          if (!(li > 0.0f)) continue;
          const float w = __builtin_amdgcn_exp2f(__builtin_fmaf(qml[2 * q], c, -mc));
          L += li * w;
          const float4 o4 = reinterpret_cast<const float4*>(sV[hg * nparts + i])[fi];
          acc.x += o4.x * w;
          acc.y += o4.y * w;
          acc.z += o4.z * w;
          acc.w += o4.w * w;
        }
      }
      float4 v;
      v.x = L > 0.0f ? acc.x / L : 0.0f;
      v.y = L > 0.0f ? acc.y / L : 0.0f;
      v.z = L > 0.0f ? acc.z / L : 0.0f;
      v.w = L > 0.0f ? acc.w / L : 0.0f;
      const int b0 = bk0 / a.Hkv, kv0 = bk0 % a.Hkv;
      *reinterpret_cast<float4*>(a.o + ((int64_t)b0 * a.Hq + kv0 * G + q) * D + d) = v;
    }
    return;
  }
  // partial outputs (unnormalized O, m in x units, full l) for mxfa_decode_combine
  if (qvalid) {
    float* po = a.part_o + (bh * nparts + part) * D;
#pragma unroll
    for (int dt = 0; dt < D / 32; dt++)
#pragma unroll
      for (int g = 0; g < 4; g++)
        *reinterpret_cast<float4*>(po + dt * 32 + 8 * g + 4 * h) =
            make_float4(st.o[dt][4 * g], st.o[dt][4 * g + 1], st.o[dt][4 * g + 2], st.o[dt][4 * g + 3]);
    if (h == 0) {
      a.part_ml[(bh * nparts + part) * 2] = st.m;
      a.part_ml[(bh * nparts + part) * 2 + 1] = l;
    }
  }
}

// Decode partials of mxfa_decode_noalloc: one array per device, in this code object, so that
// callers that cannot allocate (graph capture, serving loops) need no workspace.  The host
// takes its device address from the loaded module (hipModuleGetGlobal) once per device and
// passes that address to the kernels as part_o / part_ml, like a caller's workspace; the
// partials of a call are written before they are read, so nothing needs clearing, and calls
// that overlap on one device share (and race on) the array.
__device__ __attribute__((used, aligned(256))) uint8_t mxfa_decode_scratch[MXFA_DECODE_SCRATCH_BYTES];

// D = 256 holds its O accumulators, Q fragments and a block of K and V codes in flight in
// about 400 registers: one workgroup (one wave per SIMD) per CU.
#define MXFA_DECODE_SPLIT(D, SC, PR, VBLK, NAME)                                                   \
  extern "C" __global__ void __launch_bounds__(256, D == 256 ? 1 : 2) NAME(FaArgs a) {             \
    decode_split_impl<D, SC, PR, VBLK>(a);                                                         \
  }
#define MXFA_DECODE_ALL(D)                                                                          \
  MXFA_DECODE_SPLIT(D, false, P_R1, false, mxfa_decode_d##D)                                       \
  MXFA_DECODE_SPLIT(D, true, P_R1, false, mxfa_decode_d##D##_softcap)                              \
  MXFA_DECODE_SPLIT(D, false, P_R2, false, mxfa_decode_d##D##_r2)                                  \
  MXFA_DECODE_SPLIT(D, true, P_R2, false, mxfa_decode_d##D##_softcap_r2)                           \
  /* block-packed E3M2 V (read as the fp6 operand) */                                              \
  MXFA_DECODE_SPLIT(D, false, P_R1, true, mxfa_decode_d##D##_blk)                                  \
  MXFA_DECODE_SPLIT(D, true, P_R1, true, mxfa_decode_d##D##_softcap_blk)                           \
  MXFA_DECODE_SPLIT(D, false, P_R2, true, mxfa_decode_d##D##_r2_blk)                               \
  MXFA_DECODE_SPLIT(D, true, P_R2, true, mxfa_decode_d##D##_softcap_r2_blk)
MXFA_DECODE_ALL(64)
MXFA_DECODE_ALL(128)
MXFA_DECODE_ALL(256)

// Merge nparts partials per (b, query head) in part order: O = sum_i O_i 2^{(m_i - M) c} / sum_i l_i 2^{(m_i - M) c}.
// One workgroup of D threads per query head.
extern "C" __global__ void __launch_bounds__(256) mxfa_decode_combine(FaArgs a) {
  const int64_t bh = blockIdx.x;
  const int d = threadIdx.x;
  const int D = blockDim.x;
  const int nparts = a.n_qblk;
  const float c = a.cap_log2 > 0.0f ? 1.0f : a.c_log2;
  const float* ml = a.part_ml + bh * nparts * 2;
  float M = -INFINITY;
  for (int i = 0; i < nparts; i++)
    if (ml[2 * i + 1] > 0.0f) M = fmaxf(M, ml[2 * i]);
  float L = 0.0f, acc = 0.0f;
  if (M != -INFINITY) {
    const float mc = M * c;
    for (int i = 0; i < nparts; i++) {
      float li = ml[2 * i + 1];
      if (!(li > 0.0f)) continue;
      float w = __builtin_amdgcn_exp2f(__builtin_fmaf(ml[2 * i], c, -mc));
      L += li * w;
      acc += a.part_o[(bh * nparts + i) * D + d] * w;
    }
  }
  a.o[bh * D + d] = L > 0.0f ? acc / L : 0.0f;
}

// ---------------------------------------------------------------------------
// MX GEMM: C [M][N] fp32 = sum over 32-groups g of K of 2^(SA[g][m] + SB[g][n] - 254) *
// A[m][k] B[k][n], the operand layout of the reference's MX GEMM (A [M][K] and B [K][N]
// codes, SA [K/32][M], SB [K/32][N]), on the scaled MXFP8 MFMA with fp32 accumulation.
// Workgroup = NW waves and a 256 x 256 tile of C; the waves form 2 x NW/2, and wave
// (wr, wc) owns rows 128 wr .. +128 and 256 / (NW/2) columns as 4 x TJ MFMA tiles of
// 32 x 32 (NW = 4: one wave per SIMD, 128 x 128 per wave, accumulators in AGPRs; NW = 8:
// two per SIMD, 128 x 64).  K advances in steps of TK = 128 through two LDS stages; each
// thread stages its share of the next step in registers while the current one is
// multiplied.  A rows are read straight into the MFMA row operand; B is read with
// ds_read_b64_tr_b8 (eight k rows of one column per lane).  Rows >= M and columns >= N
// read as zero and are not stored (bounded buffer resources; M, N % 16 == 0).  The loop
// body is one basic block: E3M2 operands are a template parameter (widened to E4M3 on the
// way into LDS, exact) and the scale staging is spread over all threads without branches.
// ---------------------------------------------------------------------------
namespace gemm {
constexpr int TM = 256, TN = 256, TK = 128;
constexpr int AP = TK + 16;                // A row pitch in LDS (bytes; conflict-free b128 rows)
constexpr int BP = TN + 16;                // B row pitch (bytes)
constexpr int A_BYTES = TM * AP, B_BYTES = TK * BP;
constexpr int KB = TK / 32;                // scale blocks per step
constexpr int S_BYTES = KB * (TM + TN);    // SA [KB][TM] then SB [KB][TN]
}  // namespace gemm

template <int NW> struct GemmCfg {
  static constexpr int NT = 64 * NW;                               // threads per workgroup
  static constexpr int CH = gemm::TM * gemm::TK / 16 / NT;         // 16-byte chunks of A (and of B) per thread
  static constexpr int SPT = gemm::S_BYTES / NT;                   // scale bytes per thread per step
  static constexpr int WCN = NW / 2;                               // wave columns
  static constexpr int TJ = gemm::TN / WCN / 32;                   // 32-column MFMA tiles per wave
  static_assert(NW == 4 || NW == 8, "waves per workgroup");
  static_assert(SPT == 4 || SPT == 8, "scale staging");
};

template <int NW> struct GemmStage {
  v4i a[GemmCfg<NW>::CH];                  // A: 256 rows x TK B
  v4i b[GemmCfg<NW>::CH];                  // B: TK rows x 256 B
  uint32_t s[GemmCfg<NW>::SPT / 4];        // SPT scale codes (first half of the threads SA, second SB)
};

struct GemmRes {
  __amdgpu_buffer_rsrc_t a;                // rows m0 .. M of A
  const uint8_t* sbase;                    // SA or SB (uniform per wave)
  int sdim;                                // M or N
  uint32_t svoff;                          // offset of the thread's scale codes within a k-step
};

template <int NW>
__device__ __forceinline__ void gemm_load_scales(GemmStage<NW>& r, __amdgpu_buffer_rsrc_t rs, uint32_t voff, int soff) {
  if constexpr (GemmCfg<NW>::SPT == 4) {
    r.s[0] = __builtin_amdgcn_raw_buffer_load_b32(rs, voff, soff, 0);
  } else {
    const auto t = __builtin_amdgcn_raw_buffer_load_b64(rs, voff, soff, 0);
    r.s[0] = t[0];
    r.s[1] = t[1];
  }
}

// Everything at k >= K reads as zero (E8M0 code 0 = 2^-127 scales, so the part of a step
// past K when K % TK == 64 adds exact zeros): A chunks past K get an offset outside the
// resource, the B and scale resources end at K.
template <int NW>
__device__ __forceinline__ void gemm_load(GemmStage<NW>& r, const GemmArgs& g, const GemmRes& res, int n0, int k0,
                                          int tid) {
  using namespace gemm;
  using C = GemmCfg<NW>;
  const int krem = max(0, min(TK, g.K - k0));                   // rows of this step below K
  const __amdgpu_buffer_rsrc_t rb = buf_rsrc(g.b, (int64_t)k0 * g.N, (int64_t)krem * g.N);
#pragma unroll
  for (int i = 0; i < C::CH; i++) {
    const int c = tid + C::NT * i;
    const int row = c / (TK / 16), col = (c % (TK / 16)) * 16;  // A chunk: row, 16-byte column
    r.a[i] = __builtin_amdgcn_raw_buffer_load_b128(res.a, col < krem ? (uint32_t)(row * g.K + k0 + col) : 0x80000000u,
                                                   0, 0);
    const int kr = c >> 4, bc = (c & 15) * 16;                   // B chunk: k row, column
    const uint32_t bo = n0 + bc < g.N ? (uint32_t)(kr * g.N + n0 + bc) : 0x80000000u;
    r.b[i] = __builtin_amdgcn_raw_buffer_load_b128(rb, bo, 0, 0);
  }
  gemm_load_scales<NW>(r, buf_rsrc(res.sbase, (int64_t)(k0 / 32) * res.sdim, (int64_t)(krem / 32) * res.sdim),
                       res.svoff, 0);
}

// When K % TK == 0 every step is whole: each thread's load offsets are fixed for the
// whole K loop and the step enters as the scalar offset of the loads (k0 for A, k0 N for
// B, k0 / 32 times M or N for the scales), so a step costs no address arithmetic.  Every
// enabled load stays inside its operand (k0 <= K - TK); disabled ones (columns >= N,
// scale columns past M or N) get a vector offset past every resource and read 0, and A
// rows >= M are past the tile's resource.
template <int NW> struct GemmOff {
  uint32_t a[GemmCfg<NW>::CH];             // row K + column of the thread's A chunks
  uint32_t b[GemmCfg<NW>::CH];             // k row N + n0 + column of its B chunks
  __amdgpu_buffer_rsrc_t rb, rs;           // all of B, all of SA or SB
};

template <int NW>
__device__ __forceinline__ GemmOff<NW> gemm_offsets(const GemmArgs& g, const GemmRes& res, int n0, int tid) {
  using namespace gemm;
  using C = GemmCfg<NW>;
  GemmOff<NW> o;
#pragma unroll
  for (int i = 0; i < C::CH; i++) {
    const int c = tid + C::NT * i;
    o.a[i] = (uint32_t)((c / (TK / 16)) * g.K + (c % (TK / 16)) * 16);
    const int kr = c >> 4, bc = (c & 15) * 16;
    o.b[i] = n0 + bc < g.N ? (uint32_t)(kr * g.N + n0 + bc) : 0x80000000u;
  }
  o.rb = buf_rsrc(g.b, 0, (int64_t)g.K * g.N);
  o.rs = buf_rsrc(res.sbase, 0, (int64_t)(g.K / 32) * res.sdim);
  return o;
}

template <int NW>
__device__ __forceinline__ void gemm_load_whole(GemmStage<NW>& r, const GemmRes& res, const GemmOff<NW>& o, int k0,
                                                int N) {
#pragma unroll
  for (int i = 0; i < GemmCfg<NW>::CH; i++) {
    r.a[i] = __builtin_amdgcn_raw_buffer_load_b128(res.a, o.a[i], k0, 0);
    r.b[i] = __builtin_amdgcn_raw_buffer_load_b128(o.rb, o.b[i], k0 * N, 0);
  }
  gemm_load_scales<NW>(r, o.rs, res.svoff, (k0 / 32) * res.sdim);
}

template <int NW, int AE3, int BE3>
__device__ __forceinline__ void gemm_store(const GemmStage<NW>& r, uint8_t* sA, uint8_t* sB, uint8_t* sS, int tid) {
  using namespace gemm;
  using C = GemmCfg<NW>;
#pragma unroll
  for (int i = 0; i < C::CH; i++) {
    const int c = tid + C::NT * i;
    v4i va = r.a[i], vb = r.b[i];
    if (AE3) {
#pragma unroll
      for (int w = 0; w < 4; w++) va[w] = (int)e3m2x4_to_e4m3x4((uint32_t)va[w]);
    }
    if (BE3) {
#pragma unroll
      for (int w = 0; w < 4; w++) vb[w] = (int)e3m2x4_to_e4m3x4((uint32_t)vb[w]);
    }
    *reinterpret_cast<v4i*>(sA + (c / (TK / 16)) * AP + (c % (TK / 16)) * 16) = va;
    *reinterpret_cast<v4i*>(sB + (c >> 4) * BP + (c & 15) * 16) = vb;
  }
  if constexpr (C::SPT == 4)
    *reinterpret_cast<uint32_t*>(sS + 4 * tid) = r.s[0];
  else
    *reinterpret_cast<uint2*>(sS + 8 * tid) = make_uint2(r.s[0], r.s[1]);
}

// One k-step of the wave's 4 x TJ MFMA tiles from one LDS stage.
template <int NW>
__device__ __forceinline__ void gemm_mma(v16f (&acc)[4][GemmCfg<NW>::TJ], const uint8_t* sA, const uint8_t* sB,
                                         const uint8_t* sS, int wr, int wc, int lane) {
  using namespace gemm;
  constexpr int TJ = GemmCfg<NW>::TJ;
  const int r = lane & 31, h = lane >> 5, l16 = lane & 15, g16 = lane >> 4;
  // operands: A row tile i (rows 128 wr + 32 i + r, k = 16 h .. and 32 + 16 h ..), B
  // column tile j (column 32 TJ wc + 32 j + 16 (g16 & 1) + l16, k rows via transposed reads)
  // With two waves per SIMD the wave raises its priority from its first MFMA to the end of
  // the step, so that the one feeding the matrix pipe issues first while the other reads
  // its operands (measured +2% on the c3 QKV shape; prefill is slower with it).
  bool first = NW == 8;
#pragma unroll
  for (int kh = 0; kh < TK / 64; kh++) {                // 64-k halves of the step
    v8i bo[TJ];
    int bsc[TJ];
#pragma unroll
    for (int j = 0; j < TJ; j++) {
      const int ncol = 32 * TJ * wc + 32 * j + 16 * (g16 & 1) + 8 * (l16 & 1);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int krow = 64 * kh + 32 * (q >> 1) + 16 * h + 8 * (q & 1) + (l16 >> 1);
        v2i t = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(sB + krow * BP + ncol));
        bo[j][2 * q] = t[0];
        bo[j][2 * q + 1] = t[1];
      }
      bsc[j] = sS[KB * TM + (2 * kh + h) * TN + 32 * TJ * wc + 32 * j + r];
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int row = 128 * wr + 32 * i + r;
      const v4i lo = *reinterpret_cast<const v4i*>(sA + row * AP + 64 * kh + 16 * h);
      const v4i hi = *reinterpret_cast<const v4i*>(sA + row * AP + 64 * kh + 32 + 16 * h);
      const v8i ao = cat44(lo, hi);
      const int asc = sS[(2 * kh + h) * TM + row];
      if (first) {
        __builtin_amdgcn_s_setprio(1);
        first = false;
      }
#pragma unroll
      for (int j = 0; j < TJ; j++) acc[i][j] = mfma_mx(ao, bo[j], acc[i][j], asc, bsc[j]);
    }
  }
  if (NW == 8) __builtin_amdgcn_s_setprio(0);
}

template <int NW, int AE3, int BE3>
__device__ __forceinline__ void gemm_impl(const GemmArgs& g) {
  using namespace gemm;
  using C = GemmCfg<NW>;
  constexpr int TJ = C::TJ;
  __shared__ __attribute__((aligned(16))) uint8_t sA[2][A_BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t sB[2][B_BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t sS[2][S_BYTES];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // XCD-aware grouped order.  Workgroup lin runs on XCD lin % 8, which takes a contiguous
  // run of tile indices; tiles are numbered in groups of GM tile rows, column by column
  // inside a group, so the 32 tiles one XCD holds at a time form a 4 x 8 block of C and
  // its L2 sees 4 A panels and 8 B panels per k-step (row-major order: 2 and 24).
  constexpr int GM = 4;
  const int nwg = (int)gridDim.x, lin = (int)blockIdx.x;
  const int xcd = lin & 7, per = nwg >> 3, rem = nwg & 7;
  const int item = xcd * per + min(xcd, rem) + (lin >> 3);
  const int tiles_m = (g.M + TM - 1) / TM;
  const int group = item / (GM * g.tiles_n), first = group * GM, gm = min(GM, tiles_m - first);
  const int in_group = item - group * GM * g.tiles_n;
  const int m0 = (first + in_group % gm) * TM, n0 = (in_group / gm) * TN;
  const int wr = wave / C::WCN, wc = wave % C::WCN;

  GemmRes res;
  res.a = buf_rsrc(g.a, (int64_t)m0 * g.K, (int64_t)(g.M - m0) * g.K);
  {
    // thread t of the first (second) half of the workgroup stages scale codes
    // [k0/32 + kb][c0 + SPT cp .. + SPT] of SA (SB); its LDS bytes are SPT t ..
    constexpr int SPT = C::SPT, HALF = C::NT / 2;
    const bool is_a = wave < NW / 2;                 // wave-uniform: the scale resource stays scalar
    const int t = tid % HALF, kb = t / (256 / SPT), cp = t % (256 / SPT);
    res.sbase = is_a ? g.sa : g.sb;
    res.sdim = is_a ? g.M : g.N;
    const int c = (is_a ? m0 : n0) + SPT * cp;
    res.svoff = c < res.sdim ? (uint32_t)(kb * res.sdim + c) : 0x80000000u;
  }

  v16f acc[4][TJ];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < TJ; j++) acc[i][j] = (v16f){};

  // One register stage: step k + 1 is loaded while step k is multiplied, then stored into
  // the other LDS stage.  Loads go out first and the MFMAs before the wait of the stores
  // (the scheduler otherwise sinks the loads between the MFMAs to save registers).
  const int nk = (g.K + TK - 1) / TK;
  GemmStage<NW> st;
  gemm_load<NW>(st, g, res, n0, 0, tid);
  gemm_store<NW, AE3, BE3>(st, sA[0], sB[0], sS[0], tid);
  __syncthreads();
  if (g.K % TK == 0) {
    const GemmOff<NW> o = gemm_offsets<NW>(g, res, n0, tid);
    for (int kt = 0; kt < nk; kt++) {
      const int buf = kt & 1;
      // the last step reloads itself (in bounds; the stage is never multiplied)
      gemm_load_whole<NW>(st, res, o, min(kt + 1, nk - 1) * TK, g.N);
      __builtin_amdgcn_sched_barrier(0);
      gemm_mma<NW>(acc, sA[buf], sB[buf], sS[buf], wr, wc, lane);
      __builtin_amdgcn_sched_barrier(0);
      gemm_store<NW, AE3, BE3>(st, sA[buf ^ 1], sB[buf ^ 1], sS[buf ^ 1], tid);
      __syncthreads();
    }
  } else {
    for (int kt = 0; kt < nk; kt++) {
      const int buf = kt & 1;
      gemm_load<NW>(st, g, res, n0, (kt + 1) * TK, tid);
      __builtin_amdgcn_sched_barrier(0);
      gemm_mma<NW>(acc, sA[buf], sB[buf], sS[buf], wr, wc, lane);
      __builtin_amdgcn_sched_barrier(0);
      gemm_store<NW, AE3, BE3>(st, sA[buf ^ 1], sB[buf ^ 1], sS[buf ^ 1], tid);
      __syncthreads();
    }
  }

  // C tile: lane l, register v of tile (i, j) -> row 128 wr + 32 i + 8 (v / 4) + 4 h + v % 4,
  // column 32 TJ wc + 32 j + r.  Rows >= M fall outside the tile's resource; columns >= N
  // get an offset outside every resource.  ES = bytes per C element (4 fp32, 2 bf16).
  const int r = lane & 31, h = lane >> 5;
  const int rows = min(TM, g.M - m0);
  const int ES = g.c_bf16 ? 2 : 4;
  const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(g.c + (int64_t)m0 * g.N * ES), 0, (int)(uint32_t)((int64_t)rows * g.N * ES), 0x00020000);
#pragma unroll
  for (int j = 0; j < TJ; j++) {
    const int n = n0 + 32 * TJ * wc + 32 * j + r;
    const uint32_t cb = n < g.N ? (uint32_t)((128 * wr + 4 * h) * g.N + n) * (uint32_t)ES : 0xfffffff0u;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const uint32_t off = n < g.N ? cb + (uint32_t)((32 * i + 8 * (v >> 2) + (v & 3)) * g.N) * (uint32_t)ES : cb;
        if (g.c_bf16)
          __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (__bf16)acc[i][j][v]), rc, off, 0, 0);
        else
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[i][j][v]), rc, off, 0, 0);
      }
  }
}

// MX GEMM with LDS DMA staging (E4M3 x E4M3, K % TK == 0).  The next step's A, B and scale
// tiles are brought into the other LDS stage by buffer_load ... lds while this step multiplies:
// no staging registers and no LDS stores by the waves.  A DMA instruction writes 64 lanes x 16
// bytes contiguously, so the tiles are unpadded and their 16-byte chunks are XOR-swizzled
// instead (each lane fetches the global chunk that belongs at its LDS position):
//   A (rows of TK = 128 bytes): chunk c of row r at chunk c ^ ((r >> 1) & 7) -- a ds_read_b128 of
//     16 consecutive rows at one chunk covers all 64 banks;
//   B (k rows of 256 bytes): chunk c of row k at chunk c ^ 2 (k & 7) -- the ds_read_b64_tr_b8
//     reads (8 consecutive k rows x two adjacent chunks per 32 lanes) cover all 64 banks.
// The scale tile [KB][TM + TN] needs no swizzle (dword DMA, one 256-byte row per instruction).
template <int NW>
__device__ __forceinline__ int gemm_dma_swa(int row) { return (row >> 1) & 7; }
__device__ __forceinline__ int gemm_dma_swb(int krow) { return 2 * (krow & 7); }

template <int NW>
__device__ __forceinline__ void gemm_mma_dma(v16f (&acc)[4][GemmCfg<NW>::TJ], const uint8_t* sA, const uint8_t* sB,
                                             const uint8_t* sS, int wr, int wc, int lane) {
  using namespace gemm;
  constexpr int TJ = GemmCfg<NW>::TJ;
  const int r = lane & 31, h = lane >> 5, l16 = lane & 15, g16 = lane >> 4;
  bool first = NW == 8;
#pragma unroll
  for (int kh = 0; kh < TK / 64; kh++) {
    v8i bo[TJ];
    int bsc[TJ];
#pragma unroll
    for (int j = 0; j < TJ; j++) {
      const int ncol = 32 * TJ * wc + 32 * j + 16 * (g16 & 1) + 8 * (l16 & 1);
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int krow = 64 * kh + 32 * (q >> 1) + 16 * h + 8 * (q & 1) + (l16 >> 1);
        const int addr = krow * TN + ((((ncol >> 4) ^ gemm_dma_swb(krow))) << 4) + (ncol & 15);
        v2i t = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(sB + addr));
        bo[j][2 * q] = t[0];
        bo[j][2 * q + 1] = t[1];
      }
      bsc[j] = sS[KB * TM + (2 * kh + h) * TN + 32 * TJ * wc + 32 * j + r];
    }
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int row = 128 * wr + 32 * i + r;
      const int sw = gemm_dma_swa<NW>(row);
      const v4i lo = *reinterpret_cast<const v4i*>(sA + row * TK + (((4 * kh + h) ^ sw) << 4));
      const v4i hi = *reinterpret_cast<const v4i*>(sA + row * TK + (((4 * kh + 2 + h) ^ sw) << 4));
      const v8i ao = cat44(lo, hi);
      const int asc = sS[(2 * kh + h) * TM + row];
      if (first) {
        __builtin_amdgcn_s_setprio(1);
        first = false;
      }
#pragma unroll
      for (int j = 0; j < TJ; j++) acc[i][j] = mfma_mx(ao, bo[j], acc[i][j], asc, bsc[j]);
    }
  }
  if (NW == 8) __builtin_amdgcn_s_setprio(0);
}

// The DMA of one step into a stage: wave w issues A and B instructions w * IPW .. + IPW - 1
// (IPW = 32 / NW; instruction i covers A rows 8i .. 8i + 7 and B k rows 4i .. 4i + 3) and one
// scale row: SA row kb = w % KB (waves < NW / 2) or SB row (the others); with NW = 8 that is
// every scale row once.
struct GemmDmaLane {
  uint32_t a[2], b[2], s;   // vector offsets (A and B by instruction parity: the swizzle alternates)
};

template <int NW>
__device__ __forceinline__ void gemm_dma(const GemmArgs& g, __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb,
                                         __amdgpu_buffer_rsrc_t rs, const GemmDmaLane& dl, uint8_t* sA, uint8_t* sB,
                                         uint8_t* sS, int wave, int k0) {
  using namespace gemm;
  constexpr int IPW = 32 / NW;
#pragma unroll
  for (int q = 0; q < IPW; q++) {
    const int i = wave * IPW + q;
    dma_lds<16>(ra, sA + i * 1024, dl.a[i & 1], 8 * i * g.K + k0);
    dma_lds<16>(rb, sB + i * 1024, dl.b[i & 1], (k0 + 4 * i) * g.N);
  }
  const bool is_a = wave < NW / 2;
  const int kb = wave % KB;
  dma_lds<4>(rs, sS + (is_a ? kb * TM : KB * TM + kb * TN), dl.s, (k0 / 32 + kb) * (is_a ? g.M : g.N));
}

template <int NW>
__device__ __forceinline__ void gemm_dma_impl(const GemmArgs& g) {
  using namespace gemm;
  using C = GemmCfg<NW>;
  constexpr int TJ = C::TJ;
  static_assert(NW == 8, "DMA staging: eight waves (one scale row each)");
  __shared__ __attribute__((aligned(16))) uint8_t sA0[TM * TK];
  __shared__ __attribute__((aligned(16))) uint8_t sA1[TM * TK];
  __shared__ __attribute__((aligned(16))) uint8_t sB0[TK * TN];
  __shared__ __attribute__((aligned(16))) uint8_t sB1[TK * TN];
  __shared__ __attribute__((aligned(16))) uint8_t sS0[S_BYTES];
  __shared__ __attribute__((aligned(16))) uint8_t sS1[S_BYTES];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  constexpr int GM = 4;
  const int nwg = (int)gridDim.x, lin = (int)blockIdx.x;
  const int xcd = lin & 7, per = nwg >> 3, rem = nwg & 7;
  const int item = xcd * per + min(xcd, rem) + (lin >> 3);
  const int tiles_m = (g.M + TM - 1) / TM;
  const int group = item / (GM * g.tiles_n), first = group * GM, gm = min(GM, tiles_m - first);
  const int in_group = item - group * GM * g.tiles_n;
  const int m0 = (first + in_group % gm) * TM, n0 = (in_group / gm) * TN;
  const int wr = wave / C::WCN, wc = wave % C::WCN;

  // sources: A rows m0 .. M (rows past M read 0), all of B, SA or SB; the step enters as the
  // scalar offset
  const __amdgpu_buffer_rsrc_t ra = buf_rsrc(g.a, (int64_t)m0 * g.K, (int64_t)(g.M - m0) * g.K);
  const __amdgpu_buffer_rsrc_t rb = buf_rsrc(g.b, 0, (int64_t)g.K * g.N);
  const bool is_a = wave < NW / 2;
  const __amdgpu_buffer_rsrc_t rs = buf_rsrc(is_a ? g.sa : g.sb, 0, (int64_t)(g.K / 32) * (is_a ? g.M : g.N));
  GemmDmaLane dl;
#pragma unroll
  for (int par = 0; par < 2; par++) {
    // A instruction of parity par: lane row 8i + lane / 8, LDS chunk lane % 8
    const int ra_row = 8 * par + lane / 8, ca = (lane % 8) ^ gemm_dma_swa<NW>(ra_row);
    dl.a[par] = (uint32_t)((lane / 8) * g.K + 16 * ca);
    // B instruction of parity par: lane k row 4i + lane / 16, LDS chunk lane % 16
    const int kb_row = 4 * par + lane / 16, cb = (lane % 16) ^ gemm_dma_swb(kb_row);
    dl.b[par] = n0 + 16 * cb < g.N ? (uint32_t)((lane / 16) * g.N + n0 + 16 * cb) : 0x80000000u;
  }
  {
    const int c = (is_a ? m0 : n0) + 4 * lane;
    dl.s = c < (is_a ? g.M : g.N) ? (uint32_t)c : 0x80000000u;
  }

  v16f acc[4][TJ];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int j = 0; j < TJ; j++) acc[i][j] = (v16f){};

  const int nk = g.K / TK;
  gemm_dma<NW>(g, ra, rb, rs, dl, sA0, sB0, sS0, wave, 0);
  __builtin_amdgcn_s_waitcnt(0x0070 | 0x0f00 | 0);   // vmcnt(0)
  __syncthreads();
  auto step = [&](auto stc, int kt) {
    constexpr int ST = decltype(stc)::value;
    // the next step's tiles into the other stage (the last step reloads itself: in bounds,
    // never multiplied)
    gemm_dma<NW>(g, ra, rb, rs, dl, ST ? sA0 : sA1, ST ? sB0 : sB1, ST ? sS0 : sS1, wave, min(kt + 1, nk - 1) * TK);
    gemm_mma_dma<NW>(acc, ST ? sA1 : sA0, ST ? sB1 : sB0, ST ? sS1 : sS0, wr, wc, lane);
    __builtin_amdgcn_s_waitcnt(0x0070 | 0x0000 | 0);   // vmcnt(0) lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
  };
  for (int kt = 0; kt < nk; kt += 2) {
    step(std::integral_constant<int, 0>{}, kt);
    if (kt + 1 < nk) step(std::integral_constant<int, 1>{}, kt + 1);
  }

  const int r = lane & 31, h = lane >> 5;
  const int rows = min(TM, g.M - m0);
  const int ES = g.c_bf16 ? 2 : 4;
  const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(g.c + (int64_t)m0 * g.N * ES), 0, (int)(uint32_t)((int64_t)rows * g.N * ES), 0x00020000);
#pragma unroll
  for (int j = 0; j < TJ; j++) {
    const int n = n0 + 32 * TJ * wc + 32 * j + r;
    const uint32_t cb = n < g.N ? (uint32_t)((128 * wr + 4 * h) * g.N + n) * (uint32_t)ES : 0xfffffff0u;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const uint32_t off = n < g.N ? cb + (uint32_t)((32 * i + 8 * (v >> 2) + (v & 3)) * g.N) * (uint32_t)ES : cb;
        if (g.c_bf16)
          __builtin_amdgcn_raw_buffer_store_b16(__builtin_bit_cast(uint16_t, (__bf16)acc[i][j][v]), rc, off, 0, 0);
        else
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[i][j][v]), rc, off, 0, 0);
      }
  }
}

extern "C" __global__ void __launch_bounds__(512, 1) mxfa_gemm_dma(GemmArgs g) { gemm_dma_impl<8>(g); }

// ---------------------------------------------------------------------------
// Skinny MX GEMM (M <= 32 T rows, E4M3 x E4M3): the batched-decode projection, where the big
// kernel's 256 x 256 tiles leave the chip idle (N / 256 workgroups) and the weights B stream
// at a few percent of HBM.  One workgroup per 32-column strip of B and C (strips contiguous
// per XCD, so the four strips that share each 128-byte line of a B row share one L2).  The
// workgroup first copies all of SA and its strip of SB into LDS ((K / 32) (M + 32) bytes);
// then its four waves take the 64-k steps w, w + 4, ... and each keeps a ring of R steps of
// operands in registers, loaded R steps ahead (the loop is unrolled by R, so every ring slot
// is its own registers and every wait is a partial vmcnt):
//   B   k rows k0 + 32 q + lane / 2, 16-byte half lane % 2 of the strip (q = 0, 1; columns >= N
//       read 0), written to the wave's 2 KB LDS slab [64 k][32] for the transposed reads
//   A   row 32 i + lane % 32, bytes k0 + 16 h .. and k0 + 32 + 16 h .. (h = lane / 32): the MFMA
//       operand as it is (rows >= M read 0)
// The four partial accumulators are summed through LDS in wave order (deterministic) and C
// is stored 32 consecutive columns per 32 lanes.
// ---------------------------------------------------------------------------
constexpr int SKINNY_SCALE_BYTES = 96 * 1024;                   // (K / 32) (M + 32) at most

// Ring slots (steps in flight per wave).  Measured on M = 16 / 64 / 128 (N 6144, K 4096): 8 / 6 /
// 4 slots 11.3 / 17.0 / 25.7 us, the vmcnt limit (16 / 11 / 7) 14.1 / 18.2 / 26.4 us.
template <int T> struct SkinnyCfg {
  static constexpr int R = T == 1 ? 8 : T == 2 ? 6 : 4;
  static_assert((R - 1) * (2 + 2 * T) <= 63, "vmcnt range");
};

template <int T> struct SkinnySlot {
  v4i b[2];
  v4i a[T][2];
};

// Offsets of a disabled load get bit 31 set (arithmetic, not a select: a uniform condition
// would otherwise become a branch around the load), which puts them past every resource.
template <int T>
__device__ __forceinline__ void skinny_load(SkinnySlot<T>& sl, const GemmArgs& g, __amdgpu_buffer_rsrc_t ra,
                                            __amdgpu_buffer_rsrc_t rb, int step, bool on, int n0, int lane) {
  const int r = lane & 31, h = lane >> 5, k0 = step * 64;
  const uint32_t dis = (uint32_t)!on << 31;
#pragma unroll
  for (int q = 0; q < 2; q++) {
    const int col = n0 + 16 * (lane & 1);
    const uint32_t vo = (uint32_t)((k0 + 32 * q + (lane >> 1)) * g.N + col) | dis | ((uint32_t)(col >= g.N) << 31);
    sl.b[q] = __builtin_amdgcn_raw_buffer_load_b128(rb, vo, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < T; i++) {
    const int row = 32 * i + r;
    const uint32_t vo = (uint32_t)(row * g.K + k0 + 16 * h) | dis | ((uint32_t)(row >= g.M) << 31);
    sl.a[i][0] = __builtin_amdgcn_raw_buffer_load_b128(ra, vo, 0, 0);
    sl.a[i][1] = __builtin_amdgcn_raw_buffer_load_b128(ra, vo + 32, 0, 0);
  }
}

template <int T>
__device__ __forceinline__ void skinny_mma(v16f (&acc)[T], const SkinnySlot<T>& sl, uint8_t* slab,
                                           const uint8_t* ssa, const uint8_t* ssb, int M, int step, int lane) {
  const int r = lane & 31, h = lane >> 5, l16 = lane & 15, g16 = lane >> 4;
  // B slab [64 k][32 columns]: this lane's two 16-byte pieces, then the transposed reads
  // (one wave's LDS operations complete in order, so the previous step's reads are done)
  *reinterpret_cast<v4i*>(slab + 16 * lane) = sl.b[0];
  *reinterpret_cast<v4i*>(slab + 1024 + 16 * lane) = sl.b[1];
  v8i bo;
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int krow = 32 * (q >> 1) + 16 * h + 8 * (q & 1) + (l16 >> 1);
    const v2i t = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(slab + krow * 32 + 16 * (g16 & 1) + 8 * (l16 & 1)));
    bo[2 * q] = t[0];
    bo[2 * q + 1] = t[1];
  }
  const int sb = ssb[(2 * step + h) * 32 + r];
#pragma unroll
  for (int i = 0; i < T; i++)
    acc[i] = mfma_mx(cat44(sl.a[i][0], sl.a[i][1]), bo, acc[i], ssa[(2 * step + h) * M + 32 * i + r], sb);
}

template <int T, int... J>
__device__ __forceinline__ void skinny_round(v16f (&acc)[T], SkinnySlot<T> (&ring)[SkinnyCfg<T>::R], const GemmArgs& g,
                                             __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb, uint8_t* slab,
                                             const uint8_t* ssa, const uint8_t* ssb, int step0, int nsteps, int n0,
                                             int lane, std::integer_sequence<int, J...>) {
  constexpr int R = SkinnyCfg<T>::R;
  // slot J: multiply step step0 + 4 J, then load step step0 + 4 (J + R) into it (past the last
  // step the loads read nothing; no branch, so the waits stay partial)
  ((skinny_mma<T>(acc, ring[J], slab, ssa, ssb, g.M, step0 + 4 * J, lane),
    skinny_load<T>(ring[J], g, ra, rb, step0 + 4 * (J + R), step0 + 4 * (J + R) < nsteps, n0, lane),
    __builtin_amdgcn_sched_barrier(0)),
   ...);
}

template <int T, int... J>
__device__ __forceinline__ void skinny_tail(v16f (&acc)[T], SkinnySlot<T> (&ring)[SkinnyCfg<T>::R], uint8_t* slab,
                                            const uint8_t* ssa, const uint8_t* ssb, int M, int step0, int left,
                                            int lane, std::integer_sequence<int, J...>) {
  ((J < left ? (skinny_mma<T>(acc, ring[J], slab, ssa, ssb, M, step0 + 4 * J, lane), 0) : 0), ...);
}

template <int T>
__device__ void gemm_skinny_impl(const GemmArgs& g) {
  constexpr int R = SkinnyCfg<T>::R;
  __shared__ __attribute__((aligned(16))) uint8_t slabs[4 * 2048];
  __shared__ __attribute__((aligned(16))) uint8_t scales[SKINNY_SCALE_BYTES];
  __shared__ __attribute__((aligned(16))) float part[4 * 16 * 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nstrips = (g.N + 31) / 32;
  const int nwg = (int)gridDim.x, lin = (int)blockIdx.x;
  const int xcd = lin & 7, per = nwg >> 3, rem = nwg & 7;
  const int strip = xcd * per + min(xcd, rem) + (lin >> 3);
  if (strip >= nstrips) return;                                   // whole workgroups leave together
  const int n0 = 32 * strip;
  const __amdgpu_buffer_rsrc_t ra = buf_rsrc(g.a, 0, (int64_t)g.M * g.K);
  const __amdgpu_buffer_rsrc_t rb = buf_rsrc(g.b, 0, (int64_t)g.K * g.N);
  const int nsteps = g.K / 64, kb = g.K / 32;
  uint8_t* const slab = slabs + 2048 * wave;
  uint8_t* const ssa = scales;                                     // [K / 32][M]
  uint8_t* const ssb = scales + kb * g.M;                          // [K / 32][32]: the strip's columns

  SkinnySlot<T> ring[R];
#pragma unroll
  for (int j = 0; j < R; j++) {
    skinny_load<T>(ring[j], g, ra, rb, wave + 4 * j, wave + 4 * j < nsteps, n0, lane);
    __builtin_amdgcn_sched_barrier(0);
  }
  {
    // the scales, in batches of 8 dwords per thread (all loads of a batch before its stores;
    // M % 16 == 0 and N % 16 == 0 keep every dword aligned): SA whole, then the strip's 32
    // bytes of each SB row (columns >= N read 0)
    const __amdgpu_buffer_rsrc_t rsa = buf_rsrc(g.sa, 0, (int64_t)kb * g.M);
    const __amdgpu_buffer_rsrc_t rsb = buf_rsrc(g.sb, 0, (int64_t)kb * g.N);
    const int na = kb * g.M / 4, nb = kb * 8;
    for (int base = tid; base < na + nb; base += 256 * 8) {
      uint32_t v[8];
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int d = base + 256 * u;
        if (d < na) {
          v[u] = __builtin_amdgcn_raw_buffer_load_b32(rsa, 4 * d, 0, 0);
        } else {
          const int e = d - na, row = e >> 3, col = n0 + 4 * (e & 7);
          const uint32_t so = (uint32_t)(row * g.N + col) | ((uint32_t)(col >= g.N || e >= nb) << 31);
          v[u] = __builtin_amdgcn_raw_buffer_load_b32(rsb, so, 0, 0);
        }
      }
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int d = base + 256 * u;
        if (d < na + nb) reinterpret_cast<uint32_t*>(scales)[d] = v[u];
      }
    }
  }
  __syncthreads();

  v16f acc[T];
#pragma unroll
  for (int i = 0; i < T; i++) acc[i] = (v16f){};
  // this wave's steps: wave, wave + 4, ...; full rounds of R, then the last < R from the ring
  const int mine = nsteps > wave ? (nsteps - wave + 3) / 4 : 0;
  int step0 = wave;
  for (int round = 0; round < mine / R; round++, step0 += 4 * R)
    skinny_round<T>(acc, ring, g, ra, rb, slab, ssa, ssb, step0, nsteps, n0, lane, std::make_integer_sequence<int, R>{});
  skinny_tail<T>(acc, ring, slab, ssa, ssb, g.M, step0, mine % R, lane, std::make_integer_sequence<int, R - 1>{});
  // the four partials of each row tile, summed in wave order
#pragma unroll
  for (int i = 0; i < T; i++) {
#pragma unroll
    for (int v = 0; v < 16; v++) part[(wave * 16 + v) * 64 + lane] = acc[i][v];
    __syncthreads();
    for (int e = tid; e < 16 * 64; e += 256) {
      const int v = e / 64, L = e % 64;
      const float x = ((part[e] + part[1024 + e]) + part[2048 + e]) + part[3072 + e];
      const int row = 32 * i + 8 * (v >> 2) + 4 * (L >> 5) + (v & 3), col = n0 + (L & 31);
      if (row < g.M && col < g.N) {
        if (g.c_bf16)
          reinterpret_cast<__bf16*>(g.c)[(int64_t)row * g.N + col] = (__bf16)x;
        else
          reinterpret_cast<float*>(g.c)[(int64_t)row * g.N + col] = x;
      }
    }
    __syncthreads();
  }
}

extern "C" __global__ void __launch_bounds__(256, 1) mxfa_gemm_skinny_t1(GemmArgs g) { gemm_skinny_impl<1>(g); }
extern "C" __global__ void __launch_bounds__(256, 1) mxfa_gemm_skinny_t2(GemmArgs g) { gemm_skinny_impl<2>(g); }
extern "C" __global__ void __launch_bounds__(256, 1) mxfa_gemm_skinny_t4(GemmArgs g) { gemm_skinny_impl<4>(g); }

// Waves per GEMM workgroup; the host reads the workgroup size from the kernel's
// launch bounds (its maximum threads per block).
#ifndef MXFA_GEMM_WAVES
#define MXFA_GEMM_WAVES 8
#endif
#define MXFA_GEMM(AE, BE, NAME)                                                                         \
  extern "C" __global__ void __launch_bounds__(64 * MXFA_GEMM_WAVES, 1) NAME(GemmArgs g) {             \
    gemm_impl<MXFA_GEMM_WAVES, AE, BE>(g);                                                              \
  }
MXFA_GEMM(0, 0, mxfa_gemm)
MXFA_GEMM(1, 0, mxfa_gemm_ae3m2)
MXFA_GEMM(0, 1, mxfa_gemm_be3m2)
MXFA_GEMM(1, 1, mxfa_gemm_ae3m2_be3m2)
