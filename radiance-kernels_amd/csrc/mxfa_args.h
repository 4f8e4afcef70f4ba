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
  int B, Hq, Hkv, Sq, Sk;
  int q_pos0, window, causal, v_e3m2;
  int group;          // Hq / Hkv
  int hpw;            // prefill: query heads per workgroup
  int qpw;            // prefill: query positions per workgroup
  int n_qblk;         // prefill: query blocks; decode: number of partials per query head
  int split_len;      // decode: keys per partial (multiple of 64)
  float c_log2;       // softmax_scale * log2(e)  (no softcap)
  float sc_u;         // softmax_scale / softcap
  float cap_log2;     // softcap * log2(e) (0 = no softcap)
};
