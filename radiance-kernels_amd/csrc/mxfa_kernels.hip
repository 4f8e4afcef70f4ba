// MXFP8 flash attention for MI355X (gfx950): quantizers, prefill, split-KV decode, MX GEMM.
//
// Built with `hipcc --genco --offload-arch=gfx950` into mxfa_kernels.hsaco (one translation
// unit: this file includes the parts below) and launched by mxfa_host.cpp through
// hipModuleLaunchKernel.  Every entry point is extern "C" so the host looks it up by name.
//   k_quant.hip        MX quantizers (R1, R4), KV-cache append, synthetic inputs
//   k_attn_common.hip  MFMA wrappers, lane-pair reductions, buffer/DMA helpers, P-tile
//                      softmax/requant, the decode softmax + PV step, prefill pipeline stages
//   k_prefill.hip      bf16-K pre-pass, prefill (workspace, workspace-free, stage trace)
//   k_decode.hip       split-KV decode, partials merge
//   k_gemm.hip         MX GEMM (register-staged, LDS-DMA, skinny)
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

#include "kernel_base.h"
#include "k_quant.hip"
#include "k_attn_common.hip"
#include "k_prefill.hip"
#include "k_decode.hip"
#include "k_gemm.hip"
