// Attention building blocks shared by prefill and decode: MFMA wrappers, lane-pair
// reductions, buffer resources and LDS DMA, the P-tile softmax/requant rules
// (mxfa_softmax_requant), the decode softmax + PV step, the prefill pipeline stages
// (scores, mask, softmax, PV, O store).
#pragma once

#include "kernel_base.h"

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
