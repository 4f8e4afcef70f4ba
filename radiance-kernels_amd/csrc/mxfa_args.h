// Kernel argument block shared by the host launcher (g++) and the gfx950 kernels
// (hipcc).  Plain C layout: pointers, then 32-bit fields.
#pragma once
#include <stdint.h>

struct FaArgs {
  const uint8_t* q;
  const uint8_t* qs;
  const uint8_t* k;
  const uint8_t* ks;
  const uint8_t* v;
  const uint8_t* vs;
  float* o;
  float* part_o;      // decode: partial O  [B*Hq][nparts][D]
  float* part_ml;     // decode: partial (m, l) [B*Hq][nparts][2]
  const uint8_t* kbf; // prefill: bf16 copy of K [B][Hkv][Sk][D] (mxfa_k_to_bf16)
  const uint8_t* vws; // prefill: E4M3 copy of E3M2 V [B][Hkv][Sk][D] (mxfa_k_to_bf16), else NULL
  int B, Hq, Hkv, Sq, Sk;
  int Skc;            // keys allocated per (b, KV head) in k/ks/v/vs (>= Sk; base offsets use it)
  int q_pos0, window, causal, v_e3m2;
  int group;          // Hq / Hkv
  int hpw;            // prefill: query heads per workgroup
  int qpw;            // prefill: query positions per workgroup
  int n_qblk;         // prefill: query blocks; decode: interleaved partials per query head
  int fuse_combine;   // decode (D <= 128): the chunks of a head merge inside the workgroup
  float c_log2;       // softmax_scale * log2(e)  (no softcap)
  float sc_u;         // softmax_scale / softcap
  float cap_log2;     // softcap * log2(e) (0 = no softcap)
  // stage trace (mxfa_prefill_trace): the workgroup of item (tr_qx, tr_qy) runs alone and the
  // wave holding query rows tr_q0 .. tr_q0 + 31 of head tr_head records its stages
  float* tr_s;        // [32][Sk] scores after softcap and mask (kernel units)
  float* tr_ml;       // [n_blocks][32][2] (m, l) after each block (kernel units; l summed over the row)
  uint8_t* tr_p;      // [32][Sk] P codes
  uint8_t* tr_ps;     // [32][Sk / 32] P scale codes
  int tr_head, tr_q0, tr_qx, tr_qy;
};

// Size of the code object's device-resident decode scratch (mxfa_decode_scratch), the partials
// of mxfa_decode_noalloc: B * Hq * n_parts * (D + 2) floats at most.
#define MXFA_DECODE_SCRATCH_BYTES (16u << 20)

// MX GEMM kernel arguments: C [M][N] fp32 = A [M][K] x B [K][N] (element codes) with E8M0
// scales SA [K/32][M] and SB [K/32][N].
struct GemmArgs {
  const uint8_t* a;
  const uint8_t* sa;
  const uint8_t* b;
  const uint8_t* sb;
  uint8_t* c;         // fp32 or bf16 C [M][N]
  int M, N, K;
  int b_e3m2;         // B element codes are E3M2 (widened to E4M3 on the way to LDS)
  int a_e3m2;         // A element codes are E3M2
  int tiles_n;        // number of 256-column tiles
  int c_bf16;         // C is written as bf16 (round to nearest even)
};
