// Prefill: the bf16-K pre-pass and the prefill kernel in its workspace, workspace-free
// and stage-trace forms.
#pragma once

#include "k_attn_common.hip"

// ---------------------------------------------------------------------------
// Prefill (workspace form shown; the workspace-free form widens K in LDS instead).  The MX
// K operand is dequantized once, by mxfa_k_to_bf16, into a bf16 copy [B][Hkv][Sk][D]
// (exact: E4M3 x 2^k is a bf16 value); the prefill stages that copy and V into LDS by DMA,
// so it holds no staging registers and converts nothing: at D <= 128, 168 registers per
// lane and three 4-wave workgroups per CU (D = 256: two, with one K stage).
// With every wave issuing at most one instruction per few cycles, the third wave per SIMD
// raises the issue rate by half.  Per key block j, one barrier:
//   DMA K_bf16(j+1), V(j+1) into the other stage -> scores of j (bf16 MFMA) -> mask ->
//   softmax + P requant -> O rescale -> PV (scaled MXFP8 MFMA) -> wait, barrier.
// ---------------------------------------------------------------------------
// Workspace pre-pass: each thread converts PRE_G pieces of 8 codes (a quarter 32-block) of
// one (batch, KV head) -- blockIdx.y -- the workgroup's 256 * PRE_G consecutive pieces of
// that head, all loads issued before the stores.  A piece widens to 16 bytes of bf16, so each
// store instruction writes 1 KB of whole lines (16-byte pieces, each widened into two 16-byte
// stores 32 bytes apart, wrote every line half per instruction: 8.2 vs 7.9 us on the S = 4096
// GQA prefill).  D / 8 pieces per row (8, 16
// or 32) divides 256, so a thread's pieces share one column and step 256 / (D / 8) rows.
// Row t of head h in the copies is row h * Skc + t of the cache-strided input: the bf16 value
// of K (kbf) and, when vws is set, the E4M3 code of E3M2 V (e3m2x4_to_e4m3x4: the same
// value) -- one launch for both.
constexpr int PRE_G = 16;

extern "C" __global__ void __launch_bounds__(256) mxfa_k_to_bf16(const uint8_t* __restrict__ k,
                                                                  const uint8_t* __restrict__ ks,
                                                                  const uint8_t* __restrict__ v, int D, int Sk,
                                                                  int Skc, uint8_t* __restrict__ kbf,
                                                                  uint8_t* __restrict__ vws) {
  const int lppr = D == 256 ? 5 : D == 128 ? 4 : 3;               // log2 of pieces per row
  const int c0 = blockIdx.x * blockDim.x * PRE_G + threadIdx.x;   // piece within the head
  const int col = c0 & ((1 << lppr) - 1);
  const int rstep = (int)blockDim.x >> lppr;
  const int t0 = c0 >> lppr;
  const int64_t hq = blockIdx.y;
  int64_t so[PRE_G], doff[PRE_G];   // source and copy byte offsets of piece g (past the end: row 0)
  v2i x[PRE_G];
  float sc[PRE_G];
#pragma unroll
  for (int g = 0; g < PRE_G; g++) {
    const int t = t0 + g * rstep;
    const int64_t src = t < Sk ? hq * Skc + t : 0;
    so[g] = src * D + col * 8;
    doff[g] = (hq * Sk + t) * D + col * 8;
    x[g] = *reinterpret_cast<const v2i*>(k + so[g]);
    sc[g] = e8m0_as_float(ks[src * (D / 32) + col / 4]);
  }
#pragma unroll
  for (int g = 0; g < PRE_G; g++)
    if (t0 + g * rstep < Sk)
      *reinterpret_cast<v4i*>(kbf + doff[g] * 2) = fp8x8_to_bf16x8((uint32_t)x[g][0], (uint32_t)x[g][1], sc[g]);
  if (vws) {
#pragma unroll
    for (int g = 0; g < PRE_G; g++) x[g] = *reinterpret_cast<const v2i*>(v + so[g]);
#pragma unroll
    for (int g = 0; g < PRE_G; g++) {
      if (t0 + g * rstep < Sk) {
        v2i z;
        z[0] = (int)e3m2x4_to_e4m3x4((uint32_t)x[g][0]);
        z[1] = (int)e3m2x4_to_e4m3x4((uint32_t)x[g][1]);
        *reinterpret_cast<v2i*>(vws + doff[g]) = z;
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
