// The token reduction Pᵀ·X as device code shared by lora.hip (tn_kernel, tn_batch_kernel) and mx_gemm.hip
// (whose plain 4-wave GEMM can run a job table of these reductions in workgroups past its own tiles).  The body
// takes its LDS from the caller, so a kernel with a larger buffer of its own (the GEMM's ring) lends it instead
// of adding a second static allocation.
// Reference behaviour: the bf16 token products dB = dyᵀ·xa and dA = dxaᵀ·x of
// /root/reference/scripts/fused_mlp.py:316-318, :333 (torch GEMMs there).
#pragma once

#include "abi_common.h"
#include "mx_device.h"

namespace mxk {

constexpr int kTnTile = 32 * kTrLd;  // one per-wave [32][kTrLd] bf16 transpose tile

// bf16 elements of LDS one tn workgroup needs at rank RP: per wave an X tile and one P tile (two at RP = 64)
template <int RP>
constexpr int tn_lds_elems() {
  return 4 * kTnTile * (1 + (RP > 32 ? 2 : 1));
}

// part[c, ρ, k] = Σ_{t in chunk c} P[t, ρ] X[t, k], P [T, RP] bf16, X [T, K] bf16 (row stride ldx).  A workgroup
// of 4 waves owns 128 columns (bx) of one token chunk (by); wave w takes columns bx * 128 + 32 w .. + 31.  Per
// 32-token step the wave writes its X tile and the P tile to LDS and reads both back with k along the tokens
// (16x16x32 MFMA: A = Xᵀ rows k, B = Pᵀ as columns ρ); tokens past the chunk are zero.  `lds` holds at least
// tn_lds_elems<RP>() bf16, 16-byte aligned.
template <int RP, int kD>
__device__ __forceinline__ void tn_body(const uint16_t* __restrict__ X, int64_t ldx, const uint16_t* __restrict__ P,
                                        int T, int K, int chunk, float* __restrict__ part, int bx, int by,
                                        uint16_t* __restrict__ lds) {
  constexpr int NH = RP / 16;
  constexpr int NP = RP > 32 ? 2 : 1;  // P tiles per wave
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane((threadIdx.x >> 6) & 3), lg = lane >> 5;
  uint16_t* const xt = lds + w * kTnTile;
  uint16_t* const pt = lds + 4 * kTnTile + w * NP * kTnTile;  // pt + h * kTnTile: the wave's P tile h
  const int kb = bx * 128 + w * 32;
  const int t0 = by * chunk, t1 = min(t0 + chunk, T);
  v4f acc[2][NH];
#pragma unroll
  for (int jh = 0; jh < 2; ++jh)
#pragma unroll
    for (int h = 0; h < NH; ++h) acc[jh][h] = v4f{};
  constexpr int PW = RP / 4;  // packed words of P per lane: half of the row (RP / 2 values)
  struct Step {
    uint32_t x[8];   // X row t + l % 32, columns kb + lg*16 .. + 15
    uint32_t p[PW];  // P row t + l % 32, columns lg * RP/2 .. + RP/2 - 1
    bool ok;         // row t + l % 32 inside the chunk
  };
  auto fetch = [&](int t, Step& st) {
    const int row = t + (lane & 31);
    st.ok = row < t1;
    const int rc = min(row, T - 1);
    load16(X + (int64_t)rc * ldx + kb + lg * 16, st.x);
    const uint16_t* prow = P + (int64_t)rc * RP + lg * (RP / 2);
    if constexpr (RP == 16) {
      const uint4 v = *reinterpret_cast<const uint4*>(prow);
      st.p[0] = v.x; st.p[1] = v.y; st.p[2] = v.z; st.p[3] = v.w;
    } else {
#pragma unroll
      for (int q = 0; q < PW; q += 8) load16(prow + 2 * q, st.p + q);
    }
  };
  auto consume = [&](Step& cur) {
    // tokens past the chunk are zero (not 0 * whatever row T - 1 holds); masked here, at the use, so the
    // loads stay in flight until then
#pragma unroll
    for (int k = 0; k < 8; ++k) cur.x[k] = cur.ok ? cur.x[k] : 0u;
#pragma unroll
    for (int k = 0; k < PW; ++k) cur.p[k] = cur.ok ? cur.p[k] : 0u;
    tr_store(xt, lane, cur.x);
    // P tile row l % 32: the lane's RP/2 columns (RP = 64: lane half lg fills tile lg, columns 0..31)
    {
      uint32_t* prow = reinterpret_cast<uint32_t*>(pt + (RP > 32 ? lg * kTnTile : 0) + (lane & 31) * kTrLd) +
                       (RP > 32 ? 0 : lg * (PW));
#pragma unroll
      for (int k = 0; k < PW; k += 2) *reinterpret_cast<uint2*>(prow + k) = make_uint2(cur.p[k], cur.p[k + 1]);
    }
    const v8bf a0 = tr_operand(xt, 0, lane), a1 = tr_operand(xt, 16, lane);
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      const v8bf b = RP > 32 ? tr_operand(pt + (h >> 1) * kTnTile, (h & 1) * 16, lane) : tr_operand(pt, h * 16, lane);
      acc[0][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b, acc[0][h], 0, 0, 0);
      acc[1][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b, acc[1][h], 0, 0, 0);
    }
  };
  // Register ring of kD 32-token steps: each round but the last consumes a slot and refills it kD steps ahead,
  // unconditionally (a conditional load would make the counter waits at the loop header drain the ring); the
  // refills past the chunk reload its last step, never consumed.  kD = 1 loads each step after the previous one
  // is consumed.
  const int nsteps = (t1 - t0 + 31) / 32;
  Step ring[kD];
#pragma unroll
  for (int j = 0; j < kD; ++j) fetch(t0 + 32 * min(j, nsteps - 1), ring[j]);
  int s0 = 0;
  for (; s0 + kD < nsteps; s0 += kD) {
#pragma unroll
    for (int j = 0; j < kD; ++j) {
      consume(ring[j]);
      fetch(t0 + 32 * min(s0 + j + kD, nsteps - 1), ring[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < kD; ++j)
    if (s0 + j < nsteps) consume(ring[j]);
  // acc[jh][h] lane l: ρ = 16 h + l % 16, k = kb + 16 jh + (l / 16) * 4 + i
#pragma unroll
  for (int jh = 0; jh < 2; ++jh)
#pragma unroll
    for (int h = 0; h < NH; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rho = h * 16 + (lane & 15);
        const int k = kb + jh * 16 + (lane >> 4) * 4 + i;
        part[((int64_t)by * RP + rho) * K + k] = acc[jh][h][i];
      }
}

// The token reductions of mxfp8_lora_tn_batch (rank 16, 32 or 64 each) as one flat grid: job j owns blocks
// first[j] .. first[j + 1] - 1, `cols` = K / 128 column blocks per token chunk; every job shares T, K and the
// chunking.  kd: the ring depth (1 or 2) of tn_body.
struct TnBatch {
  const uint16_t* x[MXFP8_LORA_TN_MAX_JOBS];
  int64_t ldx[MXFP8_LORA_TN_MAX_JOBS];
  const uint16_t* p[MXFP8_LORA_TN_MAX_JOBS];
  float* part[MXFP8_LORA_TN_MAX_JOBS];
  int rp[MXFP8_LORA_TN_MAX_JOBS];
  int first[MXFP8_LORA_TN_MAX_JOBS + 1];
  int n, T, K, chunk, cols, kd;
  int wide;  // some job has rank 64
};

// LDS the batch body needs: ranks 16 and 32 (kWide false), or also 64 (kWide true)
template <bool kWide>
constexpr int tn_batch_lds_elems() {
  return tn_lds_elems<kWide ? 64 : 32>();
}

// Block b of the batch's flat grid.  Rank 64 is compiled only with kWide (its LDS is half again as large).
template <int kD, bool kWide>
__device__ __forceinline__ void tn_batch_block(const TnBatch& a, int b, uint16_t* __restrict__ lds) {
  int j = 0;
  while (j + 1 < a.n && a.first[j + 1] <= b) ++j;
  const int l = b - a.first[j], bx = l % a.cols, by = l / a.cols;
  if (a.rp[j] == 16) tn_body<16, kD>(a.x[j], a.ldx[j], a.p[j], a.T, a.K, a.chunk, a.part[j], bx, by, lds);
  else if (!kWide || a.rp[j] == 32)
    tn_body<32, kD>(a.x[j], a.ldx[j], a.p[j], a.T, a.K, a.chunk, a.part[j], bx, by, lds);
  else
    tn_body<64, kD>(a.x[j], a.ldx[j], a.p[j], a.T, a.K, a.chunk, a.part[j], bx, by, lds);
}

// The sums of the batch's jobs in one flat grid (job j: blocks first[j] .. first[j + 1] - 1).
struct TnSumBatch {
  const float* part[MXFP8_LORA_TN_MAX_JOBS];
  int rp[MXFP8_LORA_TN_MAX_JOBS];
  float scale[MXFP8_LORA_TN_MAX_JOBS];
  int transpose[MXFP8_LORA_TN_MAX_JOBS];
  int out_f32[MXFP8_LORA_TN_MAX_JOBS];
  void* out[MXFP8_LORA_TN_MAX_JOBS];
  int first[MXFP8_LORA_TN_MAX_JOBS + 1];
  int n, chunks, K;
};

// Host side (lora.hip): check mxfp8_lora_tn_batch's jobs and fill both launch tables; nb / ns = the blocks of
// the reduction and of the sum grids.  Returns MXFP8_OK, or MXFP8_ERR_ARG with the message set under `who`.
int tn_batch_tables(const char* who, const mxfp8_lora_tn_job* jobs, int64_t n_jobs, int64_t T, int64_t K,
                    int64_t chunks, float* part, TnBatch& a, TnSumBatch& sa, int64_t& nb, int64_t& ns);
// Host side (lora.hip): launch the sums of a batch filled by tn_batch_tables.
int tn_sum_batch_launch(const TnSumBatch& sa, int64_t ns, hipStream_t stm, const char* who);

}  // namespace mxk
