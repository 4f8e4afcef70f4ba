/*
 * mx_oracle.h -- CPU oracle for the MXFP8 flash-attention path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of the reference's
 * MX quantization rules and of its streaming (online-softmax) MX attention
 * recurrence.  It is linked only by tests/, by __graft_entry__.smoke() and by
 * bench.py's cpu_baseline leg, always as the checker.  The product library
 * (libmxfa) never calls it.
 *
 * Reference semantics restated here (paths relative to the reference tree):
 *   - element/scale rules ("R1"): lib/golden/mx_fp_math.h:11-28 (bf16 RNE),
 *     :205-225 (E4M3 encode), :227-236 (E4M3 decode), :249-252 (E8M0),
 *     :256-264 (E3M2 decode), :266-335 (bf16 -> E3M2 code pipeline);
 *     lib/golden/mx_golden.cpp:146-190 (block-32 requant post-pass:
 *     scale = floor(log2f(amax)) - {8 | 4} + 127, clamp [0,254], amax==0 -> 0).
 *   - attention recurrence: kernels/flash_attention_mx_gemma/
 *     flash_attention_model.py:317-372 (scale -> softcap -> mask -> block max ->
 *     corr -> exp -> requant P -> PV -> rescale; deferred 1/l with l<=0 -> 0),
 *     kernels/flash_attention_mx_gqa/flash_attention_model.py:175-248 (GQA
 *     head sharing h -> h / (Hq/Hkv), causal key_pos > query_pos masking,
 *     q_pos0), kernels/flash_attention_mx_gqa/fa_gen_data.py:95-117 (Q, K
 *     blocked along D; V blocked along the key axis).
 *
 * Deliberate, documented differences from the reference's bf16 Python model
 * (whose fp8_matmul_model dependency is not vendored): arithmetic is done in
 * double and P is rounded to fp32 before requantization, because the
 * MI355X kernels compute in fp32; the P requant rule is R1 (lib/golden),
 * which is the rule the build targets, or, with p_rule = ORC_P_R2, the
 * reference device kernels' truncating rule on P rounded to bf16 (the
 * reference's P is bf16; its bf16 exp and bf16 row-sum accumulation are
 * not restated: l sums the bf16 P values in double).
 */
#ifndef MX_ORACLE_H
#define MX_ORACLE_H

#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_FMT_E4M3 0
#define ORC_FMT_E3M2 1

/* floorf(log2f(x)) for finite x > 0, bit-exact with the glibc libm that the
 * reference's lib/golden code calls (mx_fp_math.h:209, mx_golden.cpp:171).
 * Computed from the exponent plus a per-binade mantissa threshold table that
 * orc_init() derives by correctly rounding log2 to float. */
int      orc_floor_log2f(float x);
/* The derived tables, for tests: thr[E] (E = biased exponent 1..254) is the
 * smallest 23-bit mantissa at which floorf(log2f) returns e+1 (0x800000 =
 * never); sub_thr[p] is the same for subnormals whose leading bit is p. */
void     orc_log2_tables(uint32_t thr[256], uint32_t sub_thr[23]);

uint16_t orc_f32_to_bf16(float x);           /* mx_fp_math.h:11-28 */
float    orc_bf16_to_f32(uint16_t b);
uint8_t  orc_e4m3_encode(float v);           /* mx_fp_math.h:205-225 */
float    orc_e4m3_decode(uint8_t c);         /* mx_fp_math.h:227-236 */
uint8_t  orc_e3m2_encode_bf16(uint16_t b);   /* mx_fp_math.h:266-335 */
float    orc_e3m2_decode(uint8_t c);         /* mx_fp_math.h:256-264 */
double   orc_e8m0_decode(uint8_t c);         /* mx_fp_math.h:249-252 (NaN for 255) */
uint8_t  orc_scale_code(float amax, int fmt);/* mx_golden.cpp:169-174 */

/* Quantize n values (stride apart) as one MX block (n <= 32): writes codes
 * (code_stride apart) and returns the E8M0 scale code. mx_golden.cpp:162-190. */
uint8_t  orc_quantize_block(const float *v, int64_t stride, int n, int fmt,
                            uint8_t *codes, int64_t code_stride);
/* Row-blocked: scales[rows][cols/32].  Column-blocked: scales[rows/32][cols]. */
void     orc_quantize_rows(const float *x, int64_t rows, int64_t cols, int fmt,
                           uint8_t *codes, uint8_t *scales);
void     orc_quantize_cols(const float *x, int64_t rows, int64_t cols, int fmt,
                           uint8_t *codes, uint8_t *scales);
double   orc_decode_elem(uint8_t code, int fmt);

typedef struct {
  int32_t batch, num_q_heads, num_kv_heads, seq_q, seq_k, head_dim;
  int32_t causal;       /* key visible only if kpos <= qpos                         */
  int32_t q_pos0;       /* global position of query row 0                           */
  int32_t window;       /* 0 = off; else key also masked if kpos + window <= qpos   */
  float   softmax_scale;
  float   softcap;      /* 0 = off; else s <- cap*tanh(s/cap) after the scale      */
  int32_t v_fmt;        /* ORC_FMT_E4M3 / ORC_FMT_E3M2 (Q, K are always E4M3)      */
  int32_t p_rule;       /* ORC_P_R1 (lib/golden requant) / ORC_P_R2 (device "target-0") */
} orc_attn_params;

#define ORC_P_R1 0
#define ORC_P_R2 1
#define ORC_MAX_BLOCK_N 4096

/* Streaming MX attention over key blocks of block_n keys (block j covers keys
 * [j*block_n, (j+1)*block_n)).  Split-KV: n_parts > 0 makes n_parts independent
 * partials, partial i taking the blocks i, i + n_parts, i + 2 n_parts, ... (the
 * interleaved decode schedule of libmxfa); else split_len > 0 splits the keys into
 * contiguous chunks of split_len keys; partials are merged in order by log-sum-exp;
 * both 0 = one pass.  heads: optional list of nheads flattened (b*Hq+h)
 * indices to compute (others untouched); NULL = all.  Layouts:
 *   q [B][Hq][Sq][D], q_sc [B][Hq][Sq][D/32]
 *   k [B][Hkv][Sk][D], k_sc [B][Hkv][Sk][D/32]
 *   v [B][Hkv][Sk][D], v_sc [B][Hkv][Sk/32][D]
 *   o [B][Hq][Sq][D] fp32
 * Returns 0 on success, -1 on invalid arguments. */
int orc_attention(const orc_attn_params *p,
                  const uint8_t *q, const uint8_t *q_sc,
                  const uint8_t *k, const uint8_t *k_sc,
                  const uint8_t *v, const uint8_t *v_sc,
                  float *o, int block_n, int split_len, int n_parts,
                  const int32_t *heads, int nheads, int nthreads);

/* The stages of query row qi of head bh in a single streaming pass over key blocks of block_n:
 * S_out [seq_k] (scores in natural units after scale, softcap and mask, in the double the
 * recurrence uses; -inf where masked),
 * codes_out [seq_k] (P codes), scales_out [seq_k / 32] (P scale codes), ml_out
 * [ceil(seq_k / block_n)][2] (running max and sum after each block).  Returns 0 or -1. */
int orc_attention_trace(const orc_attn_params *p, const uint8_t *q, const uint8_t *q_sc,
                        const uint8_t *k, const uint8_t *k_sc, const uint8_t *v, const uint8_t *v_sc,
                        int block_n, int64_t bh, int64_t qi, double *S_out, uint8_t *codes_out,
                        uint8_t *scales_out, double *ml_out);

/* Unquantized fp64 softmax attention on the dequantized operands (no P
 * requant, no streaming): the sanity reference. Same layouts/params. */
int orc_attention_dense(const orc_attn_params *p,
                        const uint8_t *q, const uint8_t *q_sc,
                        const uint8_t *k, const uint8_t *k_sc,
                        const uint8_t *v, const uint8_t *v_sc,
                        float *o, const int32_t *heads, int nheads, int nthreads);

/* Self-checks used by the tests. */
int64_t orc_check_log2_vs_libm(uint32_t lo, uint32_t hi);
void    orc_e4m3_encode_range(uint32_t bits_lo, uint32_t count, uint8_t *out);
void    orc_e4m3_encode_array(const float *x, int64_t n, uint8_t *out);   /* orc_e4m3_encode per element */

/* Rule R4 (kernels/simt_quant/kernel.cpp:43-117, lib/golden/golden.py:129-170) */
uint8_t orc_r4_encode(float y);
uint8_t orc_r4_quantize_block(const float *v, uint8_t *codes);
void    orc_r4_quantize_rows(const float *x, int64_t rows, int64_t cols, uint8_t *codes, uint8_t *scales);
int64_t orc_r4_check(uint32_t lo, uint32_t hi, int mode);

/* Rule R2, the reference device kernels' P requant (kernels/flash_attention_mx_gqa/
 * flash_mx_impl.hpp:53-77, 366-388, 485-501): bf16 P, block exponent se = unbiased
 * exponent of the bf16 block maximum clamped to <= 0 (scale code se + 127), elements
 * truncated to 3 mantissa bits, flushed below 2^(se-6), saturating at 448 * 2^se. */
uint8_t orc_r2_encode(uint16_t bf16, int se);                 /* bf16_to_e4m3_scaled */
int     orc_r2_scale_exp(float amax);                         /* se of an fp32 block max */
uint8_t orc_r2_quantize_block(const float *p, int n, float *pb, uint8_t *codes);
void    orc_r2_encode_array(const uint16_t *b, const int32_t *se, int64_t n, uint8_t *out);
void    orc_r2_quantize_rows(const float *p, int64_t rows, int64_t cols, float *pb, uint8_t *codes,
                             uint8_t *scales);

/* MX GEMM, exact accumulation (see mx_oracle.c): A [M][K], SA [K/32][M], B [K][N],
 * SB [K/32][N] -> C [M][N] (double); abs_out (optional) = sum |term| per element. */
void orc_mx_gemm(const uint8_t *a, const uint8_t *sa, const uint8_t *b, const uint8_t *sb,
                 int64_t M, int64_t N, int64_t K, int a_fmt, int b_fmt, double *c, double *abs_out);

#ifdef __cplusplus
}
#endif
#endif
