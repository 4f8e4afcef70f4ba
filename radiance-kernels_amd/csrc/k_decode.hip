// Split-KV decode and the partials merge.
#pragma once

#include "k_attn_common.hip"

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
