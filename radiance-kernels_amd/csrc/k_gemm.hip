// MX GEMM: the register-staged and LDS-DMA tiled kernels and the skinny kernel.
#pragma once

#include "k_attn_common.hip"

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

// The MFMA operands of one step, read from LDS one MFMA pair ahead of their use: the B
// operand of a 64-k half (TJ column tiles, eight k rows per ds_read_b64_tr_b8) and the A
// operand of one 32-row tile, each with its E8M0 scales.
template <int NW> struct GemmOpB {
  v8i b[GemmCfg<NW>::TJ];
  int s[GemmCfg<NW>::TJ];
};
struct GemmOpA {
  v8i a;
  int s;
};

template <int NW>
__device__ __forceinline__ void gemm_read_b(GemmOpB<NW>& o, const uint8_t* sB, const uint8_t* sS, int kh, int wc,
                                            int lane) {
  using namespace gemm;
  constexpr int TJ = GemmCfg<NW>::TJ;
  const int r = lane & 31, h = lane >> 5, l16 = lane & 15, g16 = lane >> 4;
#pragma unroll
  for (int j = 0; j < TJ; j++) {
    const int ncol = 32 * TJ * wc + 32 * j + 16 * (g16 & 1) + 8 * (l16 & 1);
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const int krow = 64 * kh + 32 * (q >> 1) + 16 * h + 8 * (q & 1) + (l16 >> 1);
      const int addr = krow * TN + ((((ncol >> 4) ^ gemm_dma_swb(krow))) << 4) + (ncol & 15);
      v2i t = __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_v2i*)(sB + addr));
      o.b[j][2 * q] = t[0];
      o.b[j][2 * q + 1] = t[1];
    }
    o.s[j] = sS[KB * TM + (2 * kh + h) * TN + 32 * TJ * wc + 32 * j + r];
  }
}

template <int NW>
__device__ __forceinline__ void gemm_read_a(GemmOpA& o, const uint8_t* sA, const uint8_t* sS, int kh, int i, int wr,
                                            int lane) {
  using namespace gemm;
  const int r = lane & 31, h = lane >> 5;
  const int row = 128 * wr + 32 * i + r;
  const int sw = gemm_dma_swa<NW>(row);
  const v4i lo = *reinterpret_cast<const v4i*>(sA + row * TK + (((4 * kh + h) ^ sw) << 4));
  const v4i hi = *reinterpret_cast<const v4i*>(sA + row * TK + (((4 * kh + 2 + h) ^ sw) << 4));
  o.a = cat44(lo, hi);
  o.s = sS[(2 * kh + h) * TM + row];
}

// One step's MFMAs on the stage (sA, sB, sS).  On entry a holds the A operand of (k half 0,
// tile 0) and b0 the B operand of k half 0; the B operand of half 1 is read first, and each A
// operand is read while the MFMA pair before it is issued, so that a wave's MFMA chain waits
// on LDS only at the start of the tile (the other wave of the SIMD covers that).
template <int NW, typename Dma>
__device__ __forceinline__ void gemm_mma_dma(v16f (&acc)[4][GemmCfg<NW>::TJ], GemmOpA& a, const GemmOpB<NW>& b0,
                                             const uint8_t* sA, const uint8_t* sB, const uint8_t* sS, int wr, int wc,
                                             int lane, const Dma& dma) {
  using namespace gemm;
  constexpr int TJ = GemmCfg<NW>::TJ;
  GemmOpB<NW> b1;
  gemm_read_b<NW>(b1, sB, sS, 1, wc, lane);
  __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int kh = 0; kh < TK / 64; kh++) {
    const GemmOpB<NW>& b = kh ? b1 : b0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      GemmOpA an;
      if (i < 3) gemm_read_a<NW>(an, sA, sS, kh, i + 1, wr, lane);
      else if (kh == 0) gemm_read_a<NW>(an, sA, sS, 1, 0, wr, lane);
      __builtin_amdgcn_sched_barrier(0);   // keep the reads ahead of the MFMAs (own registers)
#pragma unroll
      for (int j = 0; j < TJ; j++) acc[i][j] = mfma_mx(a.a, b.b[j], acc[i][j], a.s, b.s[j]);
      if (kh == 0) {
        __builtin_amdgcn_sched_barrier(0);
        dma(i);   // the next step's DMA, a quarter behind each MFMA group of the first k half
      }
      if (i < 3 || kh == 0) a = an;
    }
  }
  __builtin_amdgcn_s_setprio(0);
}

// The DMA of one step into a stage: wave w issues A and B instructions w * IPW .. + IPW - 1
// (IPW = 32 / NW; instruction i covers A rows 8i .. 8i + 7 and B k rows 4i .. 4i + 3) and SR =
// 2 KB / NW scale rows: SA rows (waves < NW / 2) or SB rows (the others), kb = (w SR + u) % KB,
// so that every scale row is loaded once.
struct GemmDmaLane {
  uint32_t a[2], b[2], s;   // vector offsets (A and B by instruction parity: the swizzle alternates)
};

// Part `part` of NP issues the wave's A and B instructions q = part IPW / NP .. and, in part 0,
// its scale rows.
template <int NW, int NP = 1>
__device__ __forceinline__ void gemm_dma(const GemmArgs& g, __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rb,
                                         __amdgpu_buffer_rsrc_t rs, const GemmDmaLane& dl, uint8_t* sA, uint8_t* sB,
                                         uint8_t* sS, int wave, int k0, int part = 0) {
  using namespace gemm;
  constexpr int IPW = 32 / NW;
  static_assert(IPW % NP == 0, "DMA parts");
#pragma unroll
  for (int q = part * (IPW / NP); q < (part + 1) * (IPW / NP); q++) {
    const int i = wave * IPW + q;
    dma_lds<16>(ra, sA + i * 1024, dl.a[i & 1], 8 * i * g.K + k0);
    dma_lds<16>(rb, sB + i * 1024, dl.b[i & 1], (k0 + 4 * i) * g.N);
  }
  constexpr int SR = 2 * KB / NW;
  const bool is_a = wave < NW / 2;
  if (part != 0) return;
#pragma unroll
  for (int u = 0; u < SR; u++) {
    const int kb = (wave * SR + u) % KB;
    dma_lds<4>(rs, sS + (is_a ? kb * TM : KB * TM + kb * TN), dl.s, (k0 / 32 + kb) * (is_a ? g.M : g.N));
  }
}

template <int NW>
__device__ __forceinline__ void gemm_dma_impl(const GemmArgs& g) {
  using namespace gemm;
  using C = GemmCfg<NW>;
  constexpr int TJ = C::TJ;
  static_assert(NW == 4 || NW == 8, "DMA staging: four or eight waves");
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
  GemmOpA a;
  GemmOpB<NW> b0;
  gemm_read_b<NW>(b0, sB0, sS0, 0, wc, lane);
  gemm_read_a<NW>(a, sA0, sS0, 0, 0, wr, lane);
  auto step = [&](auto stc, int kt) {
    constexpr int ST = decltype(stc)::value;
    // the next step's tiles into the other stage (the last step reloads itself: in bounds,
    // never multiplied)
    const int kn = min(kt + 1, nk - 1) * TK;
    auto dma = [&](int part) {
      gemm_dma<NW, 4>(g, ra, rb, rs, dl, ST ? sA0 : sA1, ST ? sB0 : sB1, ST ? sS0 : sS1, wave, kn, part);
    };
    gemm_mma_dma<NW>(acc, a, b0, ST ? sA1 : sA0, ST ? sB1 : sB0, ST ? sS1 : sS0, wr, wc, lane, dma);
    // the stage just multiplied is free and the next one has landed once every wave is here;
    // the next step's first operands are read while this step's last MFMAs run (no DMA is in
    // flight across the loop's back edge, so the compiler's per-buffer DMA tracking holds)
    __builtin_amdgcn_s_waitcnt(0x0070 | 0x0f00 | 0);   // vmcnt(0)
    __builtin_amdgcn_s_barrier();
    __asm__ volatile("" ::: "memory");                 // no LDS read moves above the barrier
    gemm_read_b<NW>(b0, ST ? sB0 : sB1, ST ? sS0 : sS1, 0, wc, lane);
    gemm_read_a<NW>(a, ST ? sA0 : sA1, ST ? sS0 : sS1, 0, 0, wr, lane);
  };
  for (int kt = 0; kt < nk; kt += 2) {
    step(std::integral_constant<int, 0>{}, kt);
    if (kt + 1 < nk) step(std::integral_constant<int, 1>{}, kt + 1);
  }

  // C through LDS: after the last step every stage is free.  Each wave stages PR rows of its
  // 128 x 32 TJ tile at a time in its own REG bytes ([PR][32 TJ] elements, row-major) and
  // stores them as 16-byte pieces, 64 lanes covering 1 KB of consecutive rows -- whole
  // 128-byte lines -- per instruction instead of one element per lane (columns >= N are not
  // stored: N % 16 == 0 keeps every piece on one side; rows >= M are past the resource).
  const int r = lane & 31, h = lane >> 5;
  const int rows = min(TM, g.M - m0);
  __syncthreads();
  constexpr int REG = 4 * TM * TK / NW;   // the four 32 KB A and B stages, split between the waves
  uint8_t* const reg = (wave < NW / 4 ? sA0 : wave < NW / 2 ? sA1 : wave < 3 * NW / 4 ? sB0 : sB1) +
                       (wave % (NW / 4)) * REG;
  auto epilogue = [&](auto es_c) {
    constexpr int ES = decltype(es_c)::value;
    constexpr int W = 32 * TJ * ES;       // bytes of one staged row
    constexpr int PR = REG / W;           // rows per pass
    constexpr int RPI = 1024 / W;         // rows per store instruction
    const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(g.c + (int64_t)m0 * g.N * ES), 0, (int)(uint32_t)((int64_t)rows * g.N * ES), 0x00020000);
#pragma unroll
    for (int p0 = 0; p0 < 128; p0 += PR) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        if (32 * i < p0 || 32 * i >= p0 + PR) continue;
#pragma unroll
        for (int j = 0; j < TJ; j++)
#pragma unroll
          for (int v = 0; v < 16; v++) {
            uint8_t* const e = reg + (32 * i - p0 + 8 * (v >> 2) + 4 * h + (v & 3)) * W + (32 * j + r) * ES;
            if constexpr (ES == 4)
              *reinterpret_cast<float*>(e) = acc[i][j][v];
            else
              *reinterpret_cast<__bf16*>(e) = (__bf16)acc[i][j][v];
          }
      }
#pragma unroll
      for (int u = 0; u < PR / RPI; u++) {
        const int lr = u * RPI + lane / (W / 16), ch = lane % (W / 16);
        const v4i x = *reinterpret_cast<const v4i*>(reg + lr * W + ch * 16);
        const int col = n0 + 32 * TJ * wc + ch * (16 / ES);
        const uint32_t off = col < g.N ? (uint32_t)((128 * wr + p0 + lr) * g.N + col) * (uint32_t)ES : 0xfffffff0u;
        __builtin_amdgcn_raw_buffer_store_b128(x, rc, off, 0, 0);
      }
    }
  };
  if (g.c_bf16)
    epilogue(std::integral_constant<int, 2>{});
  else
    epilogue(std::integral_constant<int, 4>{});
}

#ifndef MXFA_GEMM_DMA_WAVES
#define MXFA_GEMM_DMA_WAVES 8
#endif
extern "C" __global__ void __launch_bounds__(64 * MXFA_GEMM_DMA_WAVES, 1) mxfa_gemm_dma(GemmArgs g) {
  gemm_dma_impl<MXFA_GEMM_DMA_WAVES>(g);
}

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
//   A   rows 32 i + 16 q + lane / 4, bytes k0 + 16 (lane % 4) .. (q = 0, 1; rows >= M read 0):
//       whole 64-byte row pieces per four lanes, so that an instruction touches 16 rows instead
//       of 32 (the vector L1 handles one cache line per access: M = 64 17.2 -> 13.4 us in a
//       timing copy), then through the wave's LDS slab (rows 80 bytes apart) into the MFMA
//       operand layout (row lane % 32, bytes 16 h .. and 32 + 16 h .., h = lane / 32)
// The four partial accumulators are summed through LDS in wave order (deterministic) and C
// is stored 32 consecutive columns per 32 lanes.
// ---------------------------------------------------------------------------
constexpr int SKINNY_SCALE_BYTES = 96 * 1024;                   // (K / 32) (M + 32) at most

// Ring slots (steps in flight per wave).  Measured on M = 16 / 64 / 128 (N 6144, K 4096): 8 / 6 /
// 4 slots 11.3 / 17.0 / 25.7 us, the vmcnt limit (16 / 11 / 7) 14.1 / 18.2 / 26.4 us.
template <int T> struct SkinnyCfg {
  static constexpr int R = T == 1 ? 8 : T == 2 ? 6 : 4;
  static constexpr int AP = 80;                                  // A row pitch in the slab (bytes)
  static constexpr int SLAB = 2048 + T * 32 * AP;                // per-wave slab: B [64][32], A tiles
  static_assert(4 * SLAB >= 4 * 16 * 64 * 4, "the partials reuse the slabs");
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
  const int k0 = step * 64;
  const uint32_t dis = (uint32_t)!on << 31;
#pragma unroll
  for (int q = 0; q < 2; q++) {
    const int col = n0 + 16 * (lane & 1);
    const uint32_t vo = (uint32_t)((k0 + 32 * q + (lane >> 1)) * g.N + col) | dis | ((uint32_t)(col >= g.N) << 31);
    sl.b[q] = __builtin_amdgcn_raw_buffer_load_b128(rb, vo, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < T; i++)
#pragma unroll
    for (int q = 0; q < 2; q++) {
      const int row = 32 * i + 16 * q + (lane >> 2);
      const uint32_t vo = (uint32_t)(row * g.K + k0 + 16 * (lane & 3)) | dis | ((uint32_t)(row >= g.M) << 31);
      sl.a[i][q] = __builtin_amdgcn_raw_buffer_load_b128(ra, vo, 0, 0);
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
  // A tiles [32 rows][64 bytes] at row pitch AP: the loaded row pieces, then each lane's two
  // 16-byte operand pieces
  constexpr int AP = SkinnyCfg<T>::AP;
  uint8_t* const as = slab + 2048;
#pragma unroll
  for (int i = 0; i < T; i++)
#pragma unroll
    for (int q = 0; q < 2; q++)
      *reinterpret_cast<v4i*>(as + i * 32 * AP + (16 * q + (lane >> 2)) * AP + 16 * (lane & 3)) = sl.a[i][q];
  const int sb = ssb[(2 * step + h) * 32 + r];
#pragma unroll
  for (int i = 0; i < T; i++) {
    const uint8_t* ar = as + i * 32 * AP + r * AP + 16 * h;
    acc[i] = mfma_mx(cat44(*reinterpret_cast<const v4i*>(ar), *reinterpret_cast<const v4i*>(ar + 32)), bo, acc[i],
                     ssa[(2 * step + h) * M + 32 * i + r], sb);
  }
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
  __shared__ __attribute__((aligned(16))) uint8_t slabs[4 * SkinnyCfg<T>::SLAB];
  __shared__ __attribute__((aligned(16))) uint8_t scales[SKINNY_SCALE_BYTES];
  float* const part = reinterpret_cast<float*>(slabs);          // after the loop
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
  uint8_t* const slab = slabs + SkinnyCfg<T>::SLAB * wave;
  uint8_t* const ssa = scales;                                     // [K / 32][M]
  uint8_t* const ssb = scales + kb * g.M;                          // [K / 32][32]: the strip's columns

  // The scales go to LDS first: SA whole, then the strip's 32 bytes of each SB row (M % 16 ==
  // 0 and N % 16 == 0 keep every dword aligned; columns >= N read 0).  Their first batch is
  // issued before the operand ring, so that its stores wait for those loads only (vmcnt
  // counts in order) while the ring's loads stay in flight.  Loads past the arrays get bit 31
  // of the offset (no branch).
  const __amdgpu_buffer_rsrc_t rsa = buf_rsrc(g.sa, 0, (int64_t)kb * g.M);
  const __amdgpu_buffer_rsrc_t rsb = buf_rsrc(g.sb, 0, (int64_t)kb * g.N);
  const int na = kb * g.M / 4, nb = kb * 8;
  constexpr int BA = 16, BB = 8;                                   // dwords per thread per batch
  uint32_t* const sw = reinterpret_cast<uint32_t*>(scales);
  uint32_t va[BA], vb[BB];
  auto load_sa = [&](int base) {
#pragma unroll
    for (int u = 0; u < BA; u++) {
      const int d = base + tid + 256 * u;
      va[u] = __builtin_amdgcn_raw_buffer_load_b32(rsa, (uint32_t)(4 * d) | ((uint32_t)(d >= na) << 31), 0, 0);
    }
  };
  auto store_sa = [&](int base) {
#pragma unroll
    for (int u = 0; u < BA; u++)
      if (base + tid + 256 * u < na) sw[base + tid + 256 * u] = va[u];
  };
  auto load_sb = [&](int base) {
#pragma unroll
    for (int u = 0; u < BB; u++) {
      const int e = base + tid + 256 * u, row = e >> 3, col = n0 + 4 * (e & 7);
      const uint32_t so = (uint32_t)(row * g.N + col) | ((uint32_t)(col >= g.N || e >= nb) << 31);
      vb[u] = __builtin_amdgcn_raw_buffer_load_b32(rsb, so, 0, 0);
    }
  };
  auto store_sb = [&](int base) {
#pragma unroll
    for (int u = 0; u < BB; u++)
      if (base + tid + 256 * u < nb) sw[na + base + tid + 256 * u] = vb[u];
  };
  load_sa(0);
  load_sb(0);

  SkinnySlot<T> ring[R];
#pragma unroll
  for (int j = 0; j < R; j++) {
    skinny_load<T>(ring[j], g, ra, rb, wave + 4 * j, wave + 4 * j < nsteps, n0, lane);
    __builtin_amdgcn_sched_barrier(0);
  }
  store_sa(0);
  store_sb(0);
  for (int base = 256 * BA; base < na; base += 256 * BA) {
    load_sa(base);
    store_sa(base);
  }
  for (int base = 256 * BB; base < nb; base += 256 * BB) {
    load_sb(base);
    store_sb(base);
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
  // the four partials of each row tile, summed in wave order (in the slabs: every wave is past
  // its last operand reads first)
  __syncthreads();
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
