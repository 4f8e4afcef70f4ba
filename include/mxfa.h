/*
 * mxfa.h -- C ABI of the MI355X (gfx950) MXFP8 flash-attention library (libmxfa.so).
 *
 * Replaces the operator surface of ucb-bar/radiance-kernels'
 * kernels/flash_attention_mx{,_gqa,_gemma,_fp6,_stable}.  In the reference the
 * "operator" is a compile-time specialised bare-metal program: operands and
 * shape/causal/softcap/window parameters arrive as a generated header
 * (kernels/flash_attention_mx_gqa/fa_gen_data.py:119-159,
 * kernels/flash_attention_mx_gemma/fa_gen_data.py:165-182), the entry point is
 * fa_entry(arg, tid, threads, threadblock) started by mu_schedule
 * (kernels/flash_attention_mx_gqa/kernel.cpp:91-191, lib/include/mu_schedule.h:8-15)
 * and the output is bf16 O at a fixed address (kernel.cpp:46-50,115).  Here the same
 * operands (E4M3/E3M2 element codes + per-block-32 E8M0 scales) and parameters are
 * passed at run time, and O is fp32.
 *
 * Conventions
 *  - All tensors are caller-owned device memory; the library allocates nothing per
 *    call (mxfa_prefill_ws and mxfa_decode take a caller workspace).  Element codes are one byte each
 *    (E3M2 codes in the low 6 bits).  Base pointers must be 16-byte aligned.
 *  - Calls are asynchronous on `stream` (a hipStream_t; NULL = default stream) and
 *    never synchronize the host.  Results are deterministic (fixed reduction order,
 *    no floating-point atomics).  Calls are thread-safe.
 *  - Errors are returned as mxfa_status; mxfa_last_error() gives a thread-local
 *    description.  Arguments are validated before any launch.
 *
 * Layouts (B batch, Hq query heads, Hkv KV heads, Sq queries, Sk keys, D head dim):
 *   q   [B][Hq][Sq][D]   q_sc [B][Hq][Sq][D/32]     (32-blocks along D)
 *   k   [B][Hkv][Sk][D]  k_sc [B][Hkv][Sk][D/32]    (32-blocks along D)
 *   v   [B][Hkv][Sk][D]  v_sc [B][Hkv][Sk/32][D]    (32-blocks along the key axis,
 *                         the reference's V_scales[Sk/32][d], flash_attention_mx/gen_data.py:118-119)
 *   o   [B][Hq][Sq][D]   fp32
 * With kv_stride = L > Sk (a KV cache of capacity L), k/v/k_sc/v_sc are laid out with L in
 * place of Sk and only the first Sk keys of each (batch, KV head) are read.
 */
#ifndef MXFA_H
#define MXFA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MXFA_VERSION 3

typedef enum {
  MXFA_OK = 0,
  MXFA_ERR_INVALID_ARG = 1,   /* bad shape, pointer, alignment or parameter */
  MXFA_ERR_UNSUPPORTED = 2,   /* valid but not implemented (e.g. head_dim 96) */
  MXFA_ERR_HIP = 3,           /* a HIP runtime call failed */
  MXFA_ERR_MODULE = 4,        /* the gfx950 code object could not be loaded */
  MXFA_ERR_WORKSPACE = 5      /* workspace missing or too small */
} mxfa_status;

/* Element formats.  E4M3 and E3M2 hold one code per byte (E3M2 in the low 6 bits).
 * MXFA_FMT_E3M2_BLK is E3M2 packed per MX block, for V only (mxfa_quantize_cols,
 * mxfa_kv_append, mxfa_prefill, mxfa_prefill_ws, mxfa_decode, mxfa_decode_noalloc; not the
 * stage trace): the 32 codes of one column's 32-row block
 * are 24 bytes, read as one 192-bit little-endian integer of 6-bit fields: row 8g + 4a + b
 * of the block (g < 4, a < 2, b < 4) in field 16a + 4g + b, i.e. bits 6f .. 6f+5 (the first 12
 * bytes hold rows 0-3, 8-11, 16-19, 24-27, the last 12 rows 4-7, 12-15, 20-23, 28-31).  Blocks
 * laid out [mats][rows/32][cols][24] (for V: [B][Hkv][kv_stride/32][D][24]).  That is the
 * gfx950 scaled MFMA's fp6 operand in the key order of the kernels' P operand, so the
 * attention kernels copy V into LDS as it is.  Same values and scales as MXFA_FMT_E3M2. */
typedef enum { MXFA_FMT_E4M3 = 0, MXFA_FMT_E3M2 = 1, MXFA_FMT_E3M2_BLK = 2 } mxfa_fmt;

/* Requant rule of the probabilities P (the PV operand).
 *  MXFA_P_R1: lib/golden's block-32 rule (lib/golden/mx_golden.cpp:146-190): scale
 *             floor(log2f(amax)) - 8, E4M3 round-half-even saturating at 448.
 *  MXFA_P_R2: the reference device kernels' "target-0" rule
 *             (kernels/flash_attention_mx_gqa/flash_mx_impl.hpp:53-77, 366-388, 485-501):
 *             P rounded to bf16, scale = exponent of the bf16 block max clamped to <= 0,
 *             E4M3 by truncating the bf16 mantissa to 3 bits, flush below 2^(scale-6).
 *             l then sums the bf16 P. */
typedef enum { MXFA_P_R1 = 0, MXFA_P_R2 = 1 } mxfa_p_rule;

/* Attention parameters (the reference's generated FA_* defines,
 * kernels/flash_attention_mx_gemma/fa_gen_data.py:147-181). */
typedef struct {
  int32_t batch, num_q_heads, num_kv_heads; /* FA_NQ / FA_NKV; query head h reads KV head h / (Hq/Hkv) */
  int32_t seq_q, seq_k;                     /* FA_SQ / FA_SK; seq_k % 32 == 0                            */
  int32_t head_dim;                         /* FA_D: 64, 128 or 256                                       */
  int32_t causal;                           /* key kpos masked when kpos > qpos                          */
  int32_t q_pos0;                           /* FA_QPOS0: global position of query row 0 (>= 0)           */
  int32_t window;                           /* FA_WINDOW: 0 = off; else kpos masked when kpos+window <= qpos */
  float   softmax_scale;                    /* FA_SOFTMAX_SCALE (normally 1/sqrt(D))                     */
  float   softcap;                          /* FA_ATTN_SOFTCAP: 0 = off; s <- cap*tanh(s/cap) after scale */
  int32_t v_fmt;                            /* mxfa_fmt of V (Q and K are E4M3)                          */
  int32_t block_n;                          /* FA_BK: online-softmax key block; 0 = default (64)         */
  int32_t p_rule;                           /* mxfa_p_rule of P; 0 = MXFA_P_R1                           */
  int32_t kv_stride;                        /* keys allocated per (batch, KV head) in k, k_sc, v, v_sc:   */
                                            /* 0 = seq_k (dense); else >= seq_k, % 32 == 0 -- e.g. the    */
                                            /* max_len of a KV cache (keys >= seq_k are never read)       */
} mxfa_attn_params;

/* ---- MX quantization (rule of lib/golden/mx_golden.cpp:146-190 with the element
 *      codes of lib/golden/mx_fp_math.h:205-225 (E4M3) and :266-335 (E3M2)) ---- */

/* 32-blocks along each row of a rows x cols fp32 matrix (Q, K, KV-cache K).
 * codes [rows][cols], scales [rows][cols/32]; cols % 32 == 0.
 * Replaces the reference's offline mx_quantize_cols for Q and K
 * (kernels/flash_attention_mx_gqa/flash_attention_model.py:68-73, fa_gen_data.py:95-117). */
mxfa_status mxfa_quantize_rows(const float *x, int64_t rows, int32_t cols, mxfa_fmt fmt,
                               uint8_t *codes, uint8_t *scales, void *stream);

/* Rule R4, the reference's other software MX quantizer (kernels/simt_quant/kernel.cpp:43-117,
 * golden lib/golden/golden.py:129-170): per 32-block of a row, e = ceil(log2(amax / 448)),
 * E8M0 code clamp(e + 127, 0, 254), E4M3 elements round-half-even of x * 2^-e, saturating at
 * 448, subnormals kept.  Same layouts as mxfa_quantize_rows (E4M3 only). */
mxfa_status mxfa_quantize_rows_r4(const float *x, int64_t rows, int32_t cols,
                                  uint8_t *codes, uint8_t *scales, void *stream);

/* 32-blocks along the rows of each of `mats` rows x cols matrices (V, KV-cache V).
 * codes [mats][rows][cols] (MXFA_FMT_E3M2_BLK: [mats][rows/32][cols][24]),
 * scales [mats][rows/32][cols]; rows % 32 == 0, cols % 4 == 0.
 * Replaces mx_quantize_cols(V.t()) of fa_gen_data.py:103-104. */
mxfa_status mxfa_quantize_cols(const float *x, int64_t mats, int32_t rows, int32_t cols, mxfa_fmt fmt,
                               uint8_t *codes, uint8_t *scales, void *stream);

/* ---- attention ---- */

/* Prefill / full attention.  Replaces fa_entry + mu_schedule of the reference FA
 * kernels (kernels/flash_attention_mx_gqa/kernel.cpp:91-191,
 * kernels/flash_attention_mx_gemma/kernel.cpp:124-213).  Needs no workspace: every workgroup
 * widens the K blocks it reads to bf16 in LDS (exact), an E3M2 V tile is read by the PV
 * MFMA as E5M2 (the same bits, sign moved; O rescaled by 2^12, exact) and a block-packed
 * E3M2 V tile (MXFA_FMT_E3M2_BLK) as the MFMA's fp6 operand, as it is.  Three 4-wave
 * workgroups per CU for head_dim <= 128, two for 256. */
mxfa_status mxfa_prefill(const mxfa_attn_params *p,
                         const uint8_t *q, const uint8_t *q_sc,
                         const uint8_t *k, const uint8_t *k_sc,
                         const uint8_t *v, const uint8_t *v_sc,
                         float *o, void *stream);

/* Prefill with a caller workspace.  A first launch writes the bf16 value of every K element
 * (E4M3 code x 2^(scale - 127), exact in bf16) and, for E3M2 V, the E4M3 code of every V
 * element (the same value) into the workspace; the attention kernel then streams those copies
 * into LDS by DMA.  Where widening K in every workgroup costs less than one copy per call
 * (about 16 * wave-blocks < 32 * batch * num_kv_heads * seq_k, e.g. one query head per KV
 * head), the call runs mxfa_prefill's kernel instead and leaves the workspace untouched.  Same
 * inputs, outputs and O as mxfa_prefill (bit-identical with E4M3 V, where both run the same
 * arithmetic in the same order; within a few ulps with E3M2 V).  Block-packed E3M2 V needs no
 * copy: the kernel reads it from v as it is.
 * *workspace_bytes = batch * num_kv_heads * seq_k * head_dim * (2, or 3 with MXFA_FMT_E3M2 V).  A
 * workspace smaller than the plan is MXFA_ERR_WORKSPACE.
 * Replaces the same reference entry point as mxfa_prefill (kernels/flash_attention_mx_gqa/
 * kernel.cpp:91-191); the reference's matrix unit takes K's codes and scales as they are, so
 * it has no such copy: the workspace is this library's operand layout for the bf16 score MFMA. */
mxfa_status mxfa_prefill_plan(const mxfa_attn_params *p, size_t *workspace_bytes);

mxfa_status mxfa_prefill_ws(const mxfa_attn_params *p,
                            const uint8_t *q, const uint8_t *q_sc,
                            const uint8_t *k, const uint8_t *k_sc,
                            const uint8_t *v, const uint8_t *v_sc,
                            float *o, void *workspace, size_t workspace_bytes, void *stream);

/* Test entry (V as E4M3 or E3M2 codes): the stages of the workspace prefill for query rows 32 * q_tile .. + 31 of head bh
 * (= batch * num_q_heads + query head), as its own routines compute them.  Runs the one
 * workgroup of mxfa_prefill_ws that holds those rows (writing their O rows, bit-identical to
 * mxfa_prefill_ws) and records, for each key block the workgroup processes:
 *   s_out  [32][seq_k]        scores after softcap and mask (-inf masked); units: the raw
 *                             dot product q.k without softcap, softcap * tanh(.) * log2(e) with
 *   ml_out [ceil(seq_k/64)][32][2]  running max (same units) and row sum after the block
 *   p_out  [32][seq_k]        P codes (E4M3), ps_out [32][seq_k / 32] their E8M0 scale codes.
 * Entries of blocks the workgroup skips (outside the causal / window range) are not written.
 * Mirrors the reference's stage goldens (kernels/flash_attention_mx/fa_gen_goldens.py:52-58:
 * S, m, l, P codes and scales). */
mxfa_status mxfa_prefill_trace(const mxfa_attn_params *p,
                               const uint8_t *q, const uint8_t *q_sc,
                               const uint8_t *k, const uint8_t *k_sc,
                               const uint8_t *v, const uint8_t *v_sc,
                               float *o, void *workspace, size_t workspace_bytes,
                               int32_t bh, int32_t q_tile, float *s_out, float *ml_out,
                               uint8_t *p_out, uint8_t *ps_out, void *stream);

/* Split-KV decode plan for seq_q == 1 (q_pos0 is the query's position, normally
 * seq_k - 1): the 64-key blocks are dealt to *n_parts independent partials (partial i
 * takes blocks i, i + n_parts, ...; each a streaming pass) merged in order by
 * log-sum-exp.  The reference has no decode kernel; this is the same recurrence over a
 * KV cache. */
mxfa_status mxfa_decode_plan(const mxfa_attn_params *p, int32_t *n_parts, size_t *workspace_bytes);

mxfa_status mxfa_decode(const mxfa_attn_params *p,
                        const uint8_t *q, const uint8_t *q_sc,
                        const uint8_t *k_cache, const uint8_t *k_sc,
                        const uint8_t *v_cache, const uint8_t *v_sc,
                        float *o, void *workspace, size_t workspace_bytes, void *stream);

/* mxfa_decode without a workspace and without any allocation, for callers that cannot
 * allocate device memory: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.  No counterpart in the reference (it has no decode kernel and allocates
 * nothing at all).  The partials live in a device array inside the code object
 * (MXFA_DECODE_SCRATCH_BYTES = 16 MiB per device, held until the process ends); shapes whose
 * partials need more (mxfa_decode_plan's workspace_bytes) are rejected with
 * MXFA_ERR_WORKSPACE before any launch.  The code object must already be loaded on the
 * current device (mxfa_init(), or any earlier call there): otherwise MXFA_ERR_MODULE, since
 * loading it would allocate.  Same O as mxfa_decode, bit for bit.  Calls that overlap on
 * one device share the array and race: order them on one stream. */
mxfa_status mxfa_decode_noalloc(const mxfa_attn_params *p,
                                const uint8_t *q, const uint8_t *q_sc,
                                const uint8_t *k_cache, const uint8_t *k_sc,
                                const uint8_t *v_cache, const uint8_t *v_sc,
                                float *o, void *stream);

/* ---- KV cache ---- */

/* KV-cache shape for mxfa_kv_append: caches k [B][Hkv][max_len][D] + k_sc [B][Hkv][max_len][D/32],
 * v [B][Hkv][max_len][D] + v_sc [B][Hkv][max_len/32][D] (the layouts mxfa_decode reads); with
 * v_fmt MXFA_FMT_E3M2_BLK, v [B][Hkv][max_len/32][D][24], which decode and prefill read in
 * place (6 bits per V element: an E3M2-V decode moves 12% fewer bytes than with the codes
 * one per byte). */
typedef struct {
  int32_t batch, num_kv_heads;
  int32_t head_dim;                         /* multiple of 32                                 */
  int32_t max_len;                          /* cache capacity in tokens, multiple of 32       */
  int32_t v_fmt;                            /* mxfa_fmt of V (K is E4M3)                      */
} mxfa_kv_params;

/* Append n_new tokens at positions pos0 .. pos0+n_new-1 of every (batch, KV head) to an
 * MXFP8 KV cache with rule R1 (lib/golden/mx_golden.cpp:146-190): K rows per token
 * (32-blocks along D); V in 32-token blocks along the sequence (the reference's
 * V_scales[Sk/32][d], kernels/flash_attention_mx/gen_data.py:118-119).  The block still
 * open after the append is kept in fp32 in v_tail [B][Hkv][32][D] (caller-owned, kept
 * between calls) and re-quantized by the next append; positions not appended yet count
 * as 0.  After any sequence of appends (each starting at 0 or where the previous one
 * ended) the cache equals mxfa_quantize_rows / mxfa_quantize_cols of the whole sequence
 * (zero-padded to its 32-token block), bit for bit.  k_new, v_new: [B][Hkv][n_new][D] fp32.
 * Decode over L tokens straight from the cache: seq_k = L rounded up to 32, q_pos0 = L - 1
 * (the padding is masked causally), kv_stride = max_len.  The reference has no cache (its operands are baked into a header); this is the
 * producer side of the decode path. */
mxfa_status mxfa_kv_append(const mxfa_kv_params *p, const float *k_new, const float *v_new,
                           int32_t pos0, int32_t n_new, uint8_t *k_cache, uint8_t *k_sc,
                           uint8_t *v_cache, uint8_t *v_sc, float *v_tail, void *stream);

/* The attention kernels' softmax-requant step on caller scores, exposed so that it can
 * be checked bit-exactly in isolation.  Replaces fused_softmax_requant
 * (kernels/flash_attention_mx_gqa/flash_mx_impl.hpp:315-394).  s [rows][cols]
 * (cols % 32 == 0) are scores in the units of c (P = 2^((s - row_max) * c)), row_max
 * [rows] >= every score of its row.  Per 32-block of a row, with amax = 2^((block max -
 * row_max) * c) (exactly 1 where the block holds the row max):
 *   MXFA_P_R1: sc = R1 scale of amax, codes = R1 E4M3 codes of P * 2^(127 - sc);
 *   MXFA_P_R2: P rounded to bf16, sc = the bf16 exponent field of amax (<= 127), codes =
 *              R2 codes of the bf16 P with se = sc - 127.
 * Outputs p [rows][cols] (P as computed on the device, bf16-rounded under R2), codes
 * [rows][cols], scales [rows][cols/32], row_sum [rows] = sum of p. */
mxfa_status mxfa_softmax_requant(const float *s, const float *row_max, float c, int64_t rows,
                                 int32_t cols, int32_t p_rule, float *p, uint8_t *codes,
                                 uint8_t *scales, float *row_sum, void *stream);

/* ---- MX GEMM ---- */

/* Shape and element formats of mxfa_gemm (the reference's MATMUL_M/N/K defines,
 * kernels/gemm_mxgemmini/gen_mxgemm_data.py:105-107). */
typedef enum {
  MXFA_C_F32 = 0,                           /* fp32 C                                           */
  MXFA_C_BF16 = 1                           /* bf16 C (round to nearest even of the fp32 sum;   */
                                            /* the reference's C_out_bf16 format)               */
} mxfa_c_fmt;

typedef struct {
  int64_t m, n, k;                          /* m % 16 == 0, n % 16 == 0, k % 64 == 0 (> 0)     */
  int32_t a_fmt, b_fmt;                     /* mxfa_fmt of the A and B element codes            */
  int32_t c_fmt;                            /* mxfa_c_fmt of the output                         */
} mxfa_gemm_params;

/* C = A x B with MX operands in the reference MX GEMM's layouts (A_in [M][K], B_in [K][N],
 * A_scales_row [K/32][M], B_scales_col [K/32][N]; kernels/gemm_mxgemmini/gen_mxgemm_data.py:
 * 118-126, lib/golden/mx_golden.cpp:23-30): C[m][n] = sum over 32-groups g of K of
 * 2^(a_sc[g][m] + b_sc[g][n] - 254) * sum_{k in g} A[m][k] B[k][n], output c [M][N] in fp32
 * or bf16 (c_fmt; the reference's golden writes bf16, kernels/gemm_mxgemmini_ws/kernel.cpp:17).
 * Replaces the Gemmini MX GEMM driver's tile loop (lib/mxgemm/mxgemm_lib.hpp:11-250) with the
 * scaled MXFP8 MFMA (fp32 accumulation, not Gemmini's narrow accumulators).  The reference's
 * requant output (C_out + C_scales_row, rule R1) is mxfa_quantize_rows applied to c (scales
 * then [M][N/32], the transpose of C_scales_row).  M <= 128 with E4M3 operands (the
 * reference's batched-decode projections, kernels/gemv_batched_fp8_m32/64/128) runs a kernel
 * with one workgroup per 32 columns of C, the k steps split over its waves; every shape gives
 * the same C run to run. */
mxfa_status mxfa_gemm(const mxfa_gemm_params *p, const uint8_t *a, const uint8_t *a_sc,
                      const uint8_t *b, const uint8_t *b_sc, void *c, void *stream);

/* Synthetic inputs: x[i] ~ N(0,1) (counter-based hash + Box-Muller), each element
 * multiplied by outlier_mul with probability outlier_p.  Replaces make_inputs /
 * make_inputs_gqa (kernels/flash_attention_mx_gqa/flash_attention_model.py:58-65,166-172). */
mxfa_status mxfa_fill_normal(float *x, int64_t n, uint64_t seed, float outlier_p, float outlier_mul,
                             void *stream);

/* ---- library ---- */
mxfa_status mxfa_init(void);                       /* load the code object on the current device */
void        mxfa_shutdown(void);                   /* unload all modules                          */
const char *mxfa_status_string(mxfa_status st);
const char *mxfa_last_error(void);                 /* thread-local detail of the last failure      */
int32_t     mxfa_version(void);

#ifdef __cplusplus
}
#endif
#endif /* MXFA_H */
