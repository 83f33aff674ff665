// The rank-r LoRA products around the fused MLP, for gfx950: the per-step bf16 forms of the adapter
// parameters, the activation x adapter products (reduction over the model dimension), the adapter-gradient
// products (reduction over the tokens) and the final reduction of the backward kernel's partial sums.
//
// Reference (all in /root/reference/scripts/fused_mlp.py, _MLP, with bf16 torch GEMMs at fp32 accumulation):
//   :272-276  S = [A_g; A_u], b_g, b_u, a_d, b_d: bf16 copies of the fp32 adapter weights (fused_linear._cast)
//   :277      xs  = bf16(x · Sᵀ)                               [T, 2r]
//   :311-313  dxd = bf16(bf16(dy · B_d) · s_d)                 [T, r]
//   :316-318  dB_d = bf16(bf16(dyᵀ · bf16(xS_down)) · s_d)     [K, r]
//   :319-326  dxa = bf16(s · Σ partials) (gate and up scales), dB_g, dB_u = s · Σ partials (fp32), dA_d (fp32)
//   :333      dA  = bf16(dxaᵀ · x)                             [2r, K]
// Products that reduce over the model dimension read the activation once, row by row (MFMA with k along
// the row).  Products that reduce over the tokens split the tokens into chunks whose fp32 partials are added
// in chunk order by a second kernel (deterministic); inside a chunk both operands are transposed through LDS
// with ds_read_b64_tr_b16 so that k runs along the tokens.
#include <algorithm>
#include <mutex>

#include "abi_common.h"
#include "mx_device.h"
#include "tn_device.h"

using namespace mxk;

namespace {

__device__ __forceinline__ uint16_t bf(float x) { return (uint16_t)f32_to_bf16_bits(x); }

// ------------------------------------------------------------------------------------------------- prep
struct PrepArgs {
  const float *Ag, *Au, *Bg, *Bu, *Ad, *Bd;  // [r, K], [r, K], [N, r], [N, r], [r, N], [K, r] fp32
  uint16_t *S, *ST, *bg, *bu, *bgT, *buT, *ad, *adT, *bd, *bdT;
  int R, K, N;
};

// One thread per output element of: S [2r, K], Sᵀ [K, 2r], b_g, b_u [N, r], b_gᵀ, b_uᵀ [r, N], a_d [r, N],
// a_dᵀ [N, r], b_d [K, r], b_dᵀ [r, K] (round to nearest even, as Tensor.to(bfloat16)).
// I: the index type, 32-bit whenever the total fits (the per-element divisions are most of the kernel's work).
template <typename I>
__global__ __launch_bounds__(256) void prep_kernel(PrepArgs a, I total) {
  I i = (I)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const I R = a.R, K = a.K, N = a.N;
  I n = 2 * R * K;
  if (i < n) {
    const I r = i / K, k = i % K;
    a.S[i] = bf(r < R ? a.Ag[r * K + k] : a.Au[(r - R) * K + k]);
    return;
  }
  i -= n;
  if (i < n) {
    const I k = i / (2 * R), r = i % (2 * R);
    a.ST[i] = bf(r < R ? a.Ag[r * K + k] : a.Au[(r - R) * K + k]);
    return;
  }
  i -= n;
  n = N * R;
  if (i < n) { a.bg[i] = bf(a.Bg[i]); return; }
  i -= n;
  if (i < n) { a.bu[i] = bf(a.Bu[i]); return; }
  i -= n;
  if (i < n) {
    const I r = i / N, j = i % N;
    a.bgT[i] = bf(a.Bg[j * R + r]);
    return;
  }
  i -= n;
  if (i < n) {
    const I r = i / N, j = i % N;
    a.buT[i] = bf(a.Bu[j * R + r]);
    return;
  }
  i -= n;
  if (i < n) { a.ad[i] = bf(a.Ad[i]); return; }
  i -= n;
  if (i < n) {
    const I j = i / R, r = i % R;
    a.adT[i] = bf(a.Ad[r * N + j]);
    return;
  }
  i -= n;
  n = K * R;
  if (i < n) { a.bd[i] = bf(a.Bd[i]); return; }
  i -= n;
  if (i < n) {
    const I r = i / K, k = i % K;
    a.bdT[i] = bf(a.Bd[k * R + r]);
  }
}

// ------------------------------------------------------------------------------------------ transpose
// out[c, t] = x[t, c] for t < T and 0 for T <= t < Tpad; x [T, C] bf16 (row stride ldx, 16-byte aligned rows),
// out [C, Tpad].  One thread per token: it reads its row as C / 8 16-byte pieces and writes one element of each
// output row, so a wave's stores are 64 consecutive tokens (128 B) of one output row.
template <int C>
__device__ __forceinline__ void transpose_pad_body(const uint16_t* __restrict__ x, int64_t ldx, int T, int Tpad,
                                                   uint16_t* __restrict__ out, int t) {
  if (t >= Tpad) return;
  uint4 v[C / 8];
  const uint4* row = reinterpret_cast<const uint4*>(x + (int64_t)min(t, T - 1) * ldx);
#pragma unroll
  for (int j = 0; j < C / 8; ++j) v[j] = t < T ? row[j] : make_uint4(0, 0, 0, 0);
  const uint16_t* e = reinterpret_cast<const uint16_t*>(v);
#pragma unroll
  for (int c = 0; c < C; ++c) out[(int64_t)c * Tpad + t] = e[c];
}

template <int C>
__global__ __launch_bounds__(256) void transpose_pad_kernel(const uint16_t* __restrict__ x, int64_t ldx, int T,
                                                            int Tpad, uint16_t* __restrict__ out) {
  transpose_pad_body<C>(x, ldx, T, Tpad, out, blockIdx.x * 256 + threadIdx.x);
}

// A transpose job riding in another kernel's launch (mxfp8_quant_lora_tp): out [C, Tpad] = xᵀ of x [T, C], block b
// of the job covering tokens 256 b .. 256 b + 255.
struct TpJob {
  const uint16_t* x;
  int64_t ldx;
  int C;  // 16, 32 or 64; 0: no job
  uint16_t* out;
};

__device__ __forceinline__ void transpose_pad_job(const TpJob& j, int T, int Tpad, int b) {
  const int t = b * 256 + threadIdx.x;
  if (j.C == 16) transpose_pad_body<16>(j.x, j.ldx, T, Tpad, j.out, t);
  else if (j.C == 32) transpose_pad_body<32>(j.x, j.ldx, T, Tpad, j.out, t);
  else transpose_pad_body<64>(j.x, j.ldx, T, Tpad, j.out, t);
}

// ----------------------------------------------------------------------------------------- x · Wᵀ (nt)
// out[t, ρ] = bf16(X[t, :] · W[ρ, :]) (then bf16(· scale) when scale != 1), X [T, K] bf16 (row stride ldx),
// W [RP, K] bf16; optionally outT [RP, Tpad] (zero for t >= T).  Grid: Tpad / 32 row blocks, 4 waves, wave w
// summing a contiguous quarter of the K / 64 steps (w * steps / 4 up to (w + 1) * steps / 4) for the block's 32
// rows with the 32x32x16 MFMA (A = W rows ρ, B = X rows t, k along the row); the 4 quarters are added in LDS in
// a fixed order.
template <int RP>
__global__ __launch_bounds__(256) void nt_kernel(const uint16_t* __restrict__ X, int64_t ldx, const uint16_t* __restrict__ W,
                                                 int T, int Tpad, int K, float scale, uint16_t* __restrict__ out,
                                                 uint16_t* __restrict__ outT) {
  constexpr int NA = (RP + 31) / 32;  // 32-row groups of W
  __shared__ float red[4][32][RP + 1];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lg = lane >> 5;
  const int t = blockIdx.x * 32 + (lane & 31);
  const int tc = min(t, T - 1);
  const int ns = K / 64, k0 = (w * ns / 4) * 64, k1 = ((w + 1) * ns / 4) * 64;  // wave w: a contiguous quarter
  const uint16_t* xrow = X + (int64_t)tc * ldx + lg * 8;
  v16f acc[NA];
#pragma unroll
  for (int a = 0; a < NA; ++a) acc[a] = v16f{};
  for (int k = k0; k < k1; k += 64) {
    v8bf xb[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) xb[u] = load_bf8(xrow + k + 16 * u);
#pragma unroll
    for (int a = 0; a < NA; ++a) {
      const int rho = a * 32 + (lane & 31);
      const uint16_t* wrow = W + (int64_t)(rho < RP ? rho : 0) * K + lg * 8 + k;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const v8bf wv = load_bf8(wrow + 16 * u);
        acc[a] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(rho < RP ? wv : v8bf{}, xb[u], acc[a], 0, 0, 0);
      }
    }
  }
  // acc[a] lane l: t = l % 32, ρ = a*32 + (i/4)*8 + (l/32)*4 + i%4
#pragma unroll
  for (int a = 0; a < NA; ++a)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int rho = a * 32 + (i >> 2) * 8 + lg * 4 + (i & 3);
      if (rho < RP) red[w][lane & 31][rho] = acc[a][i];
    }
  __syncthreads();
  for (int idx = threadIdx.x; idx < 32 * RP; idx += 256) {
    const int tt = idx / RP, rho = idx % RP;
    const int row = blockIdx.x * 32 + tt;
    float v = round_bf16(((red[0][tt][rho] + red[1][tt][rho]) + red[2][tt][rho]) + red[3][tt][rho]);
    if (scale != 1.0f) v = round_bf16(v * scale);
    if (row < T) out[(int64_t)row * RP + rho] = bf(v);
    if (outT) outT[(int64_t)rho * Tpad + row] = row < T ? bf(v) : (uint16_t)0;
  }
}

// ------------------------------------------------------------- MX quantization fused with x · Wᵀ
// One pass over X [T, K] bf16 giving both its MX operand (codes in the MX-tiled layout and blocked scales:
// the bytes of mxfp8_quant_tiled) and out = bf16(X · Wᵀ) (then bf16(· scale) when scale != 1), W [RP, K]
// bf16, RP in {16, 32, 64}, with the zero-padded transposed copy outT.  Grid: Tpad / 32 row blocks (Tpad =
// ceil(T/128)*128, so the padded rows of the last scale tiles get scale 0), 4 waves.  The workgroup streams K
// in 128-column tiles through an LDS ring (4 stages; 3 at RP = 64) of the X tile (32 rows x 256 B) and the W
// tile (32 rows, 64 at RP = 64) filled by
// global_load_lds_dwordx4: lane i of a DMA takes row 4j + i/16 and the 16-byte chunk (i%16) ^ (row%16) of that
// row's tile piece, so a DMA reads four whole 256-byte row pieces and the LDS reads below, 16 rows at a time at
// one logical chunk, hit 16 distinct chunk positions.  Wave w takes columns 32w..32w+31 of each tile: lane l
// reads 16 contiguous values of row l%32 (columns 32w + 16(l/32) + 0..15), which with lane l^32 form one
// 32-block; it quantizes them (one 16-byte code store, the scale byte) and feeds them, as two k steps in a
// permuted column order that the W operand follows, to the 32x32x16 MFMA.  The waves' partial products are
// added in LDS in a fixed order.  Rows past T read row T - 1 (and store its codes again, the same bytes).
// Workgroups past the Tpad / 32 row blocks run the transpose job tp (mxfp8_quant_lora_tp), if any.
// Ranks 16 and 32: a 3-stage ring (48 KB) and at most 168 VGPRs, so three workgroups share a CU; against the 4-stage
// ring at two per CU, the same bytes and 0.6-0.9 us faster at configuration 3, cache warm or cold (two rounds, one
// box).  RP = 64: a 16 KB W tile, 3 stages (72 KB), two workgroups per CU.
template <int RP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(RP > 32 ? 2 : 3, 8))) void quant_lora_kernel(
    const uint16_t* __restrict__ X, int64_t ldx, int T, int K, const uint16_t* __restrict__ W,
    uint8_t* __restrict__ q, uint8_t* __restrict__ s, float scale, uint16_t* __restrict__ out,
    uint16_t* __restrict__ outT, int Tpad, const TpJob tp) {
  if ((int)blockIdx.x >= Tpad / 32) {  // the whole workgroup: before any barrier
    transpose_pad_job(tp, T, Tpad, (int)blockIdx.x - Tpad / 32);
    return;
  }
  // RP = 64: a second accumulator for W rows 32..63
  constexpr int kStages = 3, kTileB = 32 * 256, kStageB = kTileB + (RP > 32 ? 2 : 1) * kTileB;
  constexpr int kWDma = RP / 16;      // W DMAs per wave (RP rows x 256 B = RP / 4 KB per stage)
  constexpr int kDma = 2 + kWDma;     // X DMAs: 8 KB per stage, two per wave
  constexpr int kAcc = RP > 32 ? 2 : 1;
  __shared__ __attribute__((aligned(16))) uint8_t lds[kStages * kStageB];
  // The scale bytes of a step, [2 steps][32 rows][4 waves]: the 4 waves' bytes of a row are one word of the 128 x 4
  // scale tile, stored on the next step (see the loop).
  __shared__ uint32_t sbuf[2][32];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lg = lane >> 5;
  // Row block of this workgroup: the 4 row blocks of one 128-row scale tile go to workgroups b, b + 8, b + 16,
  // b + 24 of a group of 32, which run on one XCD (workgroup b runs on XCD b % 8), so each 512-byte scale tile
  // is written from one L2; a trailing partial group keeps the identity order.  Numbered in order, the four
  // writers sat on four XCDs: configuration 3, graph timing, two rounds on one box, rp 32 17.5-17.7 -> 15.8-15.9
  // us and rp 16 16.0 -> 14.5 us, the same bytes.
  int rbk = blockIdx.x;
  {
    const int b = blockIdx.x, g = b / 32;
    if ((g + 1) * 32 <= Tpad / 32) rbk = 32 * g + 4 * (b % 8) + (b / 8) % 4;
  }
  const int r0 = rbk * 32, nt = K / 128;
  // DMA sources (element pointers at tile 0)
  const int pc = lane & 15;
  const uint16_t* xsrc[2];
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    const int xr = 4 * (2 * w + jj) + (lane >> 4);
    xsrc[jj] = X + (int64_t)min(r0 + xr, T - 1) * ldx + (pc ^ (xr & 15)) * 8;
  }
  const uint16_t* wsrc[kWDma];
#pragma unroll
  for (int jj = 0; jj < kWDma; ++jj) {
    const int wr = 4 * (w * kWDma + jj) + (lane >> 4);  // < RP
    wsrc[jj] = W + (int64_t)wr * K + (pc ^ (wr & 15)) * 8;
  }
  const uint32_t lds0 = lds_addr(lds);
  auto issue = [&](int t, int slot) {  // tile t into ring slot `slot`
    const uint32_t st = lds0 + slot * kStageB;
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) dma16(xsrc[jj] + t * 128, st + (2 * w + jj) * 1024);
#pragma unroll
    for (int jj = 0; jj < kWDma; ++jj) dma16(wsrc[jj] + t * 128, st + kTileB + (w * kWDma + jj) * 1024);
  };
  const int row = lane & 31;
  const int m = r0 + row;
  const bool live = m < T;
  const int mc = live ? m : T - 1;
  const int cx = 4 * w + 2 * lg;  // the lane's first logical 16-byte chunk of a tile row
  const int sx0 = ((cx ^ (row & 15)) << 4), sx1 = (((cx + 1) ^ (row & 15)) << 4);
  v16f acc[kAcc];
#pragma unroll
  for (int h = 0; h < kAcc; ++h) acc[h] = v16f{};
  // Scale words: at step t each wave puts its 32 rows' scale bytes (block 4t + w) into sbuf[t & 1]; the next step
  // reads them beside its tile (after its barrier) and, at its end, wave w stores the words of rows 8w..8w+7 (lanes 0..7; the other lanes repeat them), one
  // 128-byte line of the scale tile, instead of every lane storing its byte (four waves x 32 bytes in 16-byte steps
  // over four lines).  The last step's words leave after the loop.
  uint8_t* const srow = s + (((int64_t)(r0 >> 7) * (K / 128)) << 9) + ((r0 & 127) >> 5) * 4;  // + tile t * 512
  const int frow = 8 * w + (lane & 7);  // the row whose word this lane stores
  auto flush = [&](int t, uint32_t word) {  // the words of step t (read from sbuf[t & 1])
    store_codes<MX_NT_FUSED>(srow + ((int64_t)t << 9) + frow * 16, word);
  };
  // Stages past the end re-load the last tile into the slot just consumed (no later step reads it).  The memory
  // counter also counts this lane's stores (two per step: the codes of tile t and the scale words of tile t - 1,
  // none at step 0), in issue order.  Behind tile t's DMAs come the (kStages - 2) later tiles' DMAs and, from step
  // kStages on, the stores of the last kStages - 1 steps; the wait leaves exactly those in flight.  (Counting the
  // DMAs alone made every step wait for the previous steps' stores to be acknowledged.)  The first kStages steps,
  // with fewer stores behind their tile, wait for the DMAs alone, which covers them.  The wait also drains this
  // wave's LDS operations, so the scale bytes written at step t - 1 are in LDS before the barrier.
  constexpr int kSt = 2;
#pragma unroll
  for (int j = 0; j < kStages - 1; ++j) issue(min(j, nt - 1), j);
  int slot = 0;
  for (int t = 0; t < nt; ++t) {
    if (t < kStages) wait_vmcnt<(kStages - 2) * kDma>();
    else wait_vmcnt<(kStages - 2) * kDma + (kStages - 1) * kSt>();
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();  // every wave's DMA of tile t landed; every wave is done with tile t - 1's slot
    issue(min(t + kStages - 1, nt - 1), slot == 0 ? kStages - 1 : slot - 1);
    const uint8_t* st = lds + slot * kStageB;
    const uint4 a = *reinterpret_cast<const uint4*>(st + row * 256 + sx0);
    const uint4 b = *reinterpret_cast<const uint4*>(st + row * 256 + sx1);
    // W row 32h + row has the swizzle of row (same row % 16).  Its fragments are read here, beside X's, so their
    // LDS latency runs under the quantization below (read after it, each MFMA waited for its own read).
    uint4 wa[kAcc], wb[kAcc];
#pragma unroll
    for (int h = 0; h < kAcc; ++h) {
      wa[h] = *reinterpret_cast<const uint4*>(st + kTileB + (32 * h + row) * 256 + sx0);
      wb[h] = *reinterpret_cast<const uint4*>(st + kTileB + (32 * h + row) * 256 + sx1);
    }
    const uint32_t sword = sbuf[(t + 1) & 1][frow];  // step t - 1's word (read at t = 0 too, unused there)
    const uint32_t v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    {
      uint4 c;
      const uint32_t e = quant16_codes(v, c);
      store_codes<MX_NT_FUSED>(q + tiled_offset(mc, (int64_t)t * 128 + 32 * w + 16 * lg, K), c);
      // both lanes of the pair write the same byte (scale 0 in the padded rows of the last scale tile)
      reinterpret_cast<uint8_t*>(sbuf[t & 1])[row * 4 + w] = live ? (uint8_t)e : (uint8_t)0;
    }
    // D[ρ][t] += W[ρ, cols] · X[t, cols] over the lane pair's 32 columns (rows ρ >= RP of the W tile: zero)
#pragma unroll
    for (int h = 0; h < kAcc; ++h) {
      const bool wl = 32 * h + row < RP;
      acc[h] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wl ? as_bf8(wa[h]) : v8bf{}, as_bf8(a), acc[h], 0, 0, 0);
      acc[h] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wl ? as_bf8(wb[h]) : v8bf{}, as_bf8(b), acc[h], 0, 0, 0);
    }
    if (t > 0) flush(t - 1, sword);
    slot = slot + 1 == kStages ? 0 : slot + 1;
  }
  wait_vmcnt<0>();       // the tail's repeated DMAs have landed: the ring can be reused
  __syncthreads();
  flush(nt - 1, sbuf[(nt - 1) & 1][frow]);
  float(*red)[32][RP + 1] = reinterpret_cast<float(*)[32][RP + 1]>(lds);  // [4 waves][32 rows t][RP]
  static_assert(4 * 32 * (RP + 1) * 4 <= kStages * kStageB, "reduction tile inside the ring");
  // acc[h] lane l: t = l % 32, ρ = 32 h + (i/4)*8 + (l/32)*4 + i%4
#pragma unroll
  for (int h = 0; h < kAcc; ++h)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int rho = 32 * h + (i >> 2) * 8 + lg * 4 + (i & 3);
      if (rho < RP) red[w][row][rho] = acc[h][i];
    }
  __syncthreads();
  for (int idx = threadIdx.x; idx < 32 * RP; idx += 256) {
    const int tt = idx / RP, rho = idx % RP;
    const int r = r0 + tt;
    float v = ((red[0][tt][rho] + red[1][tt][rho]) + red[2][tt][rho]) + red[3][tt][rho];
    v = round_bf16(v);
    if (scale != 1.0f) v = round_bf16(v * scale);
    if (r < T) out[(int64_t)r * RP + rho] = bf(v);
    if (outT) outT[(int64_t)rho * Tpad + r] = r < T ? bf(v) : (uint16_t)0;
  }
}

// ------------------------------------------------------------------ residual + rank-r epilogue
// out = bf16(x + bf16(y + scale * xa · Bᵀ)) for x, y [T, N] bf16 (row stride N), xa [T, R] (row stride ld_xa),
// B [N, R] bf16: the addmm_ of the LoRA-B product followed by the residual add, in one pass
// (/root/reference/scripts/mxfp8.py:265-293).  Grid (ceil(T / 32), N / 128), 4 waves: wave w owns the 32 x 32
// tile (rows 32b.., columns 128c + 32w..).  The rank-r product runs on the 32x32x16 MFMA with weight rows in the
// pi_col order, so each lane holds 16 contiguous columns of its row and moves x, y and out as 16-byte pieces.
template <int R, bool kVecXa>
__global__ __launch_bounds__(256) void res_lora_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ y,
                                                       const uint16_t* __restrict__ xa, int64_t ld_xa,
                                                       const uint16_t* __restrict__ B, int T, int N, float scale,
                                                       uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lg = lane >> 5;
  const int m = blockIdx.x * 32 + (lane & 31);
  const bool live = m < T;
  const int mc = live ? m : T - 1;
  const int jb = blockIdx.y * 128 + w * 32;
  const int64_t e0 = (int64_t)mc * N + jb + lg * 16;  // this lane's 16 contiguous elements
  uint32_t xv[8], yv[8];
  load16(x + e0, xv);
  load16(y + e0, yv);
  v8bf xf[R / 16], wf[R / 16];
  const int64_t wr = (int64_t)(jb + pi_col(lane & 31)) * R + lg * 8;
#pragma unroll
  for (int h = 0; h < R / 16; ++h) {
    const uint16_t* px = xa + (int64_t)mc * ld_xa + h * 16 + lg * 8;
    if constexpr (kVecXa) {
      xf[h] = load_bf8(px);
    } else {  // xa at any element offset and row stride: eight 2-byte loads
      v8s16 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = (short)px[e];
      xf[h] = __builtin_bit_cast(v8bf, v);
    }
    wf[h] = load_bf8(B + wr + h * 16);
  }
  const v16f d = lora_pi<R>(wf, xf);
  uint32_t o[8];
#pragma unroll
  for (int i = 0; i < 16; i += 2) {
    float t0 = bf16_lo(yv[i / 2]) + scale * d[i], t1 = bf16_hi(yv[i / 2]) + scale * d[i + 1];
    rnd2(t0, t1);  // t = bf16(y + scale * xa·Bᵀ)
    float o0 = bf16_lo(xv[i / 2]) + t0, o1 = bf16_hi(xv[i / 2]) + t1;
    o[i / 2] = rnd2(o0, o1);
  }
  if (live) {
    uint4* po = reinterpret_cast<uint4*>(out + e0);
    po[0] = make_uint4(o[0], o[1], o[2], o[3]);
    po[1] = make_uint4(o[4], o[5], o[6], o[7]);
  }
}

// --------------------------------------------------------------- LoRA backward of a linear: one read of dy
// For dy [T, N] bf16 (row stride ld_dy), from ONE read (/root/reference/scripts/mxfp8.py:89-262, lora_bwd):
//   kQuant: MX(dy) into columns col_tile_off*128 .. of a wider code buffer q (row stride ld_q) and its blocked
//           scales s (s_col_tiles 128-column tiles per row), byte for byte mx_quant(dy) (rows past T: scale 0);
//   kLora:  d(xa) = scale · dy · B  (B [N, R] bf16) and dB = scale · dyᵀ · xa (xa [T, R] bf16, row stride ld_xa),
//           as fp32 partial sums: part_dxa [N / 128, T, R] over each 128-column chunk (or d(xa) itself when N is
//           one chunk), part_db [rs, N, R] over each row chunk (added in order by lora_bwd_sum_kernel).
// Grid (rs, N / 128), 4 waves: the workgroup owns rows [blockIdx.x * chunk, + chunk) (clipped at Tpad, a multiple
// of 128, so the padded rows of the last scale tiles get scale 0) and 128 columns.  Each wave works alone on the
// 32-row blocks w, w + 4, ... of that range, all 128 columns: no barrier inside the loop, and d(xa) of a block is
// complete in one wave.  A block is loaded row-contiguously (16 lanes per 256-byte row piece, the next block's
// loads in flight during this one's work), stored into the wave's own LDS tile with the 16-byte chunk swizzle
// c ^ (row % 16) and read back with lane l holding 16 contiguous values of row l % 32 per 32-column group g: the
// quantizer takes them with partner lane l ^ 32, the d(xa) MFMA takes them as its B operand (A = B's rows, gathered
// once).  For dB each group's 32 x 32 tile goes through a second per-wave tile and is read back transposed
// (ds_read_b64_tr_b16), with xa, also staged per wave, read transposed: 16x16x32 MFMAs accumulate dB in registers
// over the wave's blocks; the four waves' dB are added in LDS in a fixed order at the end.
// The body takes its row chunk bx, column block by and the column block count ny as arguments (blockIdx.x,
// blockIdx.y and gridDim.y of lora_bwd_kernel; a job's share of the flat grid of lora_bwd_batch_kernel).
template <int R, bool kQuant, bool kLora>
__device__ __forceinline__ void lora_bwd_body(const uint16_t* __restrict__ dy, int64_t ld_dy, int T, int N, int Tpad,
                                              int chunk, uint8_t* __restrict__ q, int64_t ld_q,
                                              uint8_t* __restrict__ s, int64_t s_col_tiles, int col_tile_off,
                                              const uint16_t* __restrict__ xa, int64_t ld_xa,
                                              const uint16_t* __restrict__ B, float* __restrict__ part_dxa,
                                              float* __restrict__ part_db, uint16_t* __restrict__ dxa, int64_t ld_dxa,
                                              float scale, const int bx, const int by, const int ny) {
  constexpr int kTileB = 32 * 256;         // one block of one wave: 32 rows x 128 bf16
  constexpr int kRedB = kLora ? 4 * 128 * 17 * 4 : 0;  // end-of-kernel dB exchange: [wave][column][16 ρ + 1]
  constexpr int kXaL = kLora ? R / 16 : 0;  // 16-byte xa pieces per lane per block
  __shared__ __attribute__((aligned(16))) uint8_t tiles[(4 * kTileB > kRedB) ? 4 * kTileB : kRedB];
  __shared__ __attribute__((aligned(16))) uint16_t trt[4][32 * kTrLd];        // per-wave dy tile for dB
  __shared__ __attribute__((aligned(16))) uint16_t xat[4][kLora ? 32 * R : 8];  // per-wave xa tile
  __shared__ __attribute__((aligned(16))) uint8_t qtile[4][kQuant ? 32 * 128 : 16];  // per-wave block of codes
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lg = lane >> 5;
  const int r0 = bx * chunk, r1 = min(r0 + chunk, Tpad);
  const int c0 = by * 128;
  const int row = lane & 31;
  const int nblk = (r1 - r0) / 32;
  uint8_t* tile = tiles + w * kTileB;
  // loads of a block: piece j covers rows 4j + lane/16, 16-byte chunk lane%16 of the row's 256 bytes
  const int pc = lane & 15, prow = lane >> 4;
  // the wave's next two blocks, in flight (register sets ca and cb): dy pieces 0..7 and the xa pieces
  uint4 ca0, ca1, ca2, ca3, ca4, ca5, ca6, ca7, cax0, cax1;
  uint4 cb0, cb1, cb2, cb3, cb4, cb5, cb6, cb7, cbx0, cbx1;
  constexpr int xper = R / 8;  // 16-byte parts per xa row
  const uint16_t* dyc = dy + c0 + pc * 8;
  const uint16_t* xac = xa + (lane % xper) * 8;
#define LB_FETCH(b, P)                                                                                    \
  {                                                                                                       \
    const int rb_ = r0 + 32 * (b);                                                                        \
    P##0 = *reinterpret_cast<const uint4*>(dyc + (int64_t)min(rb_ + 0 + prow, T - 1) * ld_dy);            \
    P##1 = *reinterpret_cast<const uint4*>(dyc + (int64_t)min(rb_ + 4 + prow, T - 1) * ld_dy);            \
    P##2 = *reinterpret_cast<const uint4*>(dyc + (int64_t)min(rb_ + 8 + prow, T - 1) * ld_dy);            \
    P##3 = *reinterpret_cast<const uint4*>(dyc + (int64_t)min(rb_ + 12 + prow, T - 1) * ld_dy);           \
    P##4 = *reinterpret_cast<const uint4*>(dyc + (int64_t)min(rb_ + 16 + prow, T - 1) * ld_dy);           \
    P##5 = *reinterpret_cast<const uint4*>(dyc + (int64_t)min(rb_ + 20 + prow, T - 1) * ld_dy);           \
    P##6 = *reinterpret_cast<const uint4*>(dyc + (int64_t)min(rb_ + 24 + prow, T - 1) * ld_dy);           \
    P##7 = *reinterpret_cast<const uint4*>(dyc + (int64_t)min(rb_ + 28 + prow, T - 1) * ld_dy);           \
    if constexpr (kXaL >= 1)                                                                              \
      P##x0 = *reinterpret_cast<const uint4*>(xac + (int64_t)min(rb_ + lane / xper, T - 1) * ld_xa);     \
    if constexpr (kXaL >= 2)                                                                              \
      P##x1 = *reinterpret_cast<const uint4*>(xac + (int64_t)min(rb_ + 64 / xper + lane / xper, T - 1) * ld_xa); \
  }
  // d(xa) A operand: lane l holds B[n, ρ] (ρ = l % 32 < R, else 0) at the lane's columns n of group g, k step ks
  v8bf bt[4][2];
  if constexpr (kLora) {
    const int rho = row;
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        v8s16 v;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int n = c0 + 32 * g + 16 * lg + 8 * ks + e;
          v[e] = (short)B[(int64_t)n * R + (rho < R ? rho : 0)];
        }
        if (rho >= R) v = v8s16{};
        bt[g][ks] = __builtin_bit_cast(v8bf, v);
      }
  }
  v4f db[4][2][R / 16];
#pragma unroll
  for (int g = 0; g < 4; ++g)
#pragma unroll
    for (int jh = 0; jh < 2; ++jh)
#pragma unroll
      for (int h = 0; h < R / 16; ++h) db[g][jh][h] = v4f{};
  const bool direct = ny == 1;
  auto lb_block = [&](const int rb) __attribute__((always_inline)) {
    const int m = rb + row;
    const bool live = m < T;
    const int mc = live ? m : T - 1;
    v16f p = v16f{};
    uint32_t epack = 0;  // the row's four scale bytes (groups 0..3), 0 past T
    // The lane's two 16-byte pieces of group g (its first logical chunk cx = 4 g + 2 lg of the row).  Group g + 1's
    // pieces are read before group g's work, so their LDS latency runs under it (read at the top of each group,
    // every group waited for its own reads).
    auto piece = [&](int g, int k) {
      return *reinterpret_cast<const uint4*>(tile + row * 256 + (((4 * g + 2 * lg + k) ^ (row & 15)) << 4));
    };
    uint4 na = piece(0, 0), nc = piece(0, 1);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint4 a = na, c = nc;
      if (g < 3) {
        na = piece(g + 1, 0);
        nc = piece(g + 1, 1);
      }
      uint32_t v[8] = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
      if constexpr (kQuant) {
        // codes into the wave's code tile (row stride 128 B, 16-byte chunk k at k ^ (row % 8)); scales by row
        uint4 cw;
        const uint32_t e = quant16_codes(v, cw);
        epack |= (live ? e : 0u) << (8 * g);
        *reinterpret_cast<uint4*>(qtile[w] + row * 128 + (((2 * g + lg) ^ (row & 7)) << 4)) = cw;
      }
      if constexpr (kLora) {
        // d(xa) over the group's 32 columns, into D[ρ][t] (lane: t = l % 32, ρ = 8 (i / 4) + 4 (l / 32) + i % 4)
        p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bt[g][0], as_bf8(a), p, 0, 0, 0);
        p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bt[g][1], as_bf8(c), p, 0, 0, 0);
        // dB: D[n][ρ] += Σ_t dy[t, n] xa[t, ρ] over the block's rows (rows past T add nothing)
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = live ? v[k] : 0u;
        tr_store(trt[w], lane, v);
#pragma unroll
        for (int jh = 0; jh < 2; ++jh) {
          const v8bf ad = tr_operand(trt[w], jh * 16, lane);
#pragma unroll
          for (int h = 0; h < R / 16; ++h) {
            // rows past T hold row T - 1's xa: their dy is zero, so they add nothing
            const v8bf xb = tr_operand_ld(xat[w], R, h * 16, lane);
            db[g][jh][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ad, xb, db[g][jh][h], 0, 0, 0);
          }
        }
      }
    }
    if constexpr (kQuant) {
      // the block's codes as whole 128-byte row pieces: lane l takes row 8 j + l / 8, chunk l % 8 (rows past T hold
      // row T - 1's codes and store them again); the four scale bytes of a row are one word of the 128 x 4 tile
      // (lanes l and l + 32 store the same word)
      uint8_t* qrow = q + (int64_t)col_tile_off * 128 + c0 + (lane & 7) * 16;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int rr = 8 * j + (lane >> 3);
        const uint4 cw = *reinterpret_cast<const uint4*>(qtile[w] + rr * 128 + (((lane & 7) ^ (rr & 7)) << 4));
        store_codes<MX_NT_FUSED>(qrow + (int64_t)min(rb + rr, T - 1) * ld_q, cw);
      }
      store_codes<MX_NT_FUSED>(s + (((int64_t)(m >> 7) * s_col_tiles + col_tile_off + (c0 >> 7)) << 9) +
                                   (m & 31) * 16 + ((m & 127) >> 5) * 4,
                               epack);
    }
    if constexpr (kLora) {
      // rows past T computed row T - 1's values again (same inputs, same order): storing them to row T - 1
      // writes the same bytes, so every store is unconditional
      if (direct) {  // one column chunk: the sum is final (mxfp8.py:168-172, DXA_DIRECT)
        uint16_t* o = dxa + (int64_t)mc * ld_dxa;
#pragma unroll
        for (int i = 0; i < R / 2; ++i) o[(i >> 2) * 8 + lg * 4 + (i & 3)] = bf(p[i] * scale);
      } else {
        float* o = part_dxa + ((int64_t)by * T + mc) * R;
#pragma unroll
        for (int i4 = 0; i4 < R / 8; ++i4)
          *reinterpret_cast<float4*>(o + i4 * 8 + lg * 4) =
              make_float4(p[4 * i4], p[4 * i4 + 1], p[4 * i4 + 2], p[4 * i4 + 3]);
      }
    }
  };
  // LDS slot of piece j: row 4j + lane/16, physical chunk (lane%16) ^ (row%16); (4j + prow) % 16 = 4 (j % 4) + prow
  uint8_t* st0 = tile + prow * 256 + ((pc ^ prow) << 4);
  uint8_t* st1 = tile + prow * 256 + ((pc ^ (prow + 4)) << 4);
  uint8_t* st2 = tile + prow * 256 + ((pc ^ (prow + 8)) << 4);
  uint8_t* st3 = tile + prow * 256 + ((pc ^ (prow + 12)) << 4);
  // One block: stage register set P into the wave's LDS tiles, start the loads of the wave's block kAhead blocks
  // on into P (none past its last), then quantize and multiply.  Two blocks stay in flight per wave (one for
  // r = 32 with both outputs, whose accumulators leave no room for a second set).
  constexpr int kAhead = (R == 32 && kQuant && kLora) ? 4 : 8;
#define LB_BODY(b, P)                                                                                       \
  {                                                                                                         \
    *reinterpret_cast<uint4*>(st0) = P##0;                                                                  \
    *reinterpret_cast<uint4*>(st1 + 1024) = P##1;                                                           \
    *reinterpret_cast<uint4*>(st2 + 2048) = P##2;                                                           \
    *reinterpret_cast<uint4*>(st3 + 3072) = P##3;                                                           \
    *reinterpret_cast<uint4*>(st0 + 4096) = P##4;                                                           \
    *reinterpret_cast<uint4*>(st1 + 5120) = P##5;                                                           \
    *reinterpret_cast<uint4*>(st2 + 6144) = P##6;                                                           \
    *reinterpret_cast<uint4*>(st3 + 7168) = P##7;                                                           \
    if constexpr (kXaL >= 1) *reinterpret_cast<uint4*>(xat[w] + lane * 8) = P##x0;                          \
    if constexpr (kXaL >= 2) *reinterpret_cast<uint4*>(xat[w] + 512 + lane * 8) = P##x1;                    \
    if ((b) + kAhead < nblk) LB_FETCH((b) + kAhead, P)                                                      \
    lb_block(r0 + 32 * (b));                                                                                \
  }
  if constexpr (kAhead == 8) {
    if (w < nblk) LB_FETCH(w, ca)
    if (w + 4 < nblk) LB_FETCH(w + 4, cb)
    for (int b = w; b < nblk; b += 8) {
      LB_BODY(b, ca)
      if (b + 4 < nblk) LB_BODY(b + 4, cb)
    }
  } else {
    if (w < nblk) {  // the first block outside the loop: the same memory operations in flight on every entry
      LB_FETCH(w, ca)
      LB_BODY(w, ca)
    }
    for (int b = w + 4; b < nblk; b += 4) LB_BODY(b, ca)
  }
#undef LB_BODY
  if constexpr (kLora) {
    // the four waves' dB, added in wave order, 16 ρ at a time (the dy tiles are free now)
    float(*red)[128][17] = reinterpret_cast<float(*)[128][17]>(tiles);
#pragma unroll
    for (int h = 0; h < R / 16; ++h) {
      __syncthreads();
      // lane l: ρ = 16 h + l % 16, column 32 g + 16 jh + (l / 16) * 4 + i
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int jh = 0; jh < 2; ++jh)
#pragma unroll
          for (int i = 0; i < 4; ++i) red[w][32 * g + 16 * jh + (lane >> 4) * 4 + i][lane & 15] = db[g][jh][h][i];
      __syncthreads();
      for (int idx = threadIdx.x; idx < 128 * 16; idx += 256) {
        const int n = idx >> 4, rr = idx & 15;
        part_db[((int64_t)bx * N + c0 + n) * R + h * 16 + rr] =
            ((red[0][n][rr] + red[1][n][rr]) + red[2][n][rr]) + red[3][n][rr];
      }
    }
  }
}
#undef LB_FETCH

template <int R, bool kQuant, bool kLora>
__global__ __launch_bounds__(256, 2) void lora_bwd_kernel(const uint16_t* __restrict__ dy, int64_t ld_dy, int T,
                                                          int N, int Tpad, int chunk, uint8_t* __restrict__ q,
                                                          int64_t ld_q, uint8_t* __restrict__ s, int64_t s_col_tiles,
                                                          int col_tile_off, const uint16_t* __restrict__ xa,
                                                          int64_t ld_xa, const uint16_t* __restrict__ B,
                                                          float* __restrict__ part_dxa, float* __restrict__ part_db,
                                                          uint16_t* __restrict__ dxa, int64_t ld_dxa, float scale) {
  lora_bwd_body<R, kQuant, kLora>(dy, ld_dy, T, N, Tpad, chunk, q, ld_q, s, s_col_tiles, col_tile_off, xa, ld_xa, B,
                                  part_dxa, part_db, dxa, ld_dxa, scale, blockIdx.x, blockIdx.y, gridDim.y);
}

// The jobs of mxfp8_lora_bwd_batch in one flat grid: job j owns blocks first[j] .. first[j + 1] - 1, `used` row
// chunks per column block, so every layer of the group streams its dy at the same time.
struct LoraBwdBatch {
  mxfp8_lora_bwd_job job[MXFP8_LORA_BWD_MAX_JOBS];
  int first[MXFP8_LORA_BWD_MAX_JOBS + 1];
  int n, T, Tpad, chunk, used;
  uint8_t* q;
  int64_t ld_q;
  uint8_t* s;
  int64_t s_col_tiles;
};

template <int R, bool kQuant>
__global__ __launch_bounds__(256, 2) void lora_bwd_batch_kernel(const LoraBwdBatch a) {
  const int b = blockIdx.x;
  int j = 0;
  while (j + 1 < a.n && a.first[j + 1] <= b) ++j;
  const mxfp8_lora_bwd_job& jb = a.job[j];
  const int local = b - a.first[j];
  lora_bwd_body<R, kQuant, true>(static_cast<const uint16_t*>(jb.dy), jb.ld_dy, a.T, (int)jb.N, a.Tpad, a.chunk, a.q,
                                 a.ld_q, a.s, a.s_col_tiles, (int)jb.col_tile_off,
                                 static_cast<const uint16_t*>(jb.xa), jb.ld_xa, static_cast<const uint16_t*>(jb.b),
                                 jb.part_dxa, jb.part_db, static_cast<uint16_t*>(jb.dxa), jb.ld_dxa, jb.scale,
                                 local % a.used, local / a.used, (int)(jb.N / 128));
}

// 16-byte vectors of fp32 partial sums added in ascending partial order, four loads in flight at a time
__device__ __forceinline__ float4 add4(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}
// The partials are read once: streaming (non-temporal) loads.  The backward finish at configuration 3 (graph timing,
// one box, three alternating pairs, bit-identical): 13.07-13.10 us with plain loads, 12.01-12.03 us with these;
// lora_bwd's sums unchanged (23.7 / 57.9 us with the main kernel); eight loads in flight instead of four measured
// the same.  (The forward's sum_parts kernel measured slower with them: 12.8 against 11.6 us.)
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_part(const float4* p) {
  const f32x4 t = __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
  return make_float4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ float4 sum_ordered(const float4* __restrict__ p, int64_t stride, int n) {
  float4 v = ld_part(p);
  int c = 1;
  for (; c + 3 < n; c += 4) {
    const float4 x0 = ld_part(p + c * stride), x1 = ld_part(p + (c + 1) * stride), x2 = ld_part(p + (c + 2) * stride),
                 x3 = ld_part(p + (c + 3) * stride);
    v = add4(add4(add4(add4(v, x0), x1), x2), x3);
  }
  for (; c < n; ++c) v = add4(v, ld_part(p + c * stride));
  return v;
}

// dxa[t, ρ] (row stride ld_dxa) = bf16(scale · Σ_p part_dxa[p, t, ρ]) over the first nx = T·R elements (none when
// the main kernel wrote d(xa) itself) and dB[n, ρ] = scale · Σ_p part_db[p, n, ρ] (fp32) over the next N·R, partials
// added in ascending p (mxfp8.py:180-216, _sum_rows / _sum_parts).  Four consecutive elements per thread.
__device__ __forceinline__ void lora_bwd_sum_body(const float* __restrict__ part_dxa, int ncs, int64_t nx,
                                                  const float* __restrict__ part_db, int nrs, int64_t nb, int R,
                                                  float scale, uint16_t* __restrict__ dxa, int64_t ld_dxa,
                                                  float* __restrict__ dB, int64_t i) {
  if (i < nx) {
    const float4 v = sum_ordered(reinterpret_cast<const float4*>(part_dxa + i), nx / 4, ncs);
    uint16_t* o = dxa + (i / R) * ld_dxa + i % R;  // R % 4 == 0: the four share a row
    o[0] = bf(v.x * scale);
    o[1] = bf(v.y * scale);
    o[2] = bf(v.z * scale);
    o[3] = bf(v.w * scale);
    return;
  }
  i -= nx;
  if (i >= nb) return;
  const float4 v = sum_ordered(reinterpret_cast<const float4*>(part_db + i), nb / 4, nrs);
  *reinterpret_cast<float4*>(dB + i) = make_float4(v.x * scale, v.y * scale, v.z * scale, v.w * scale);
}

__global__ __launch_bounds__(256) void lora_bwd_sum_kernel(const float* __restrict__ part_dxa, int ncs, int64_t nx,
                                                           const float* __restrict__ part_db, int nrs, int64_t nb,
                                                           int R, float scale, uint16_t* __restrict__ dxa,
                                                           int64_t ld_dxa, float* __restrict__ dB) {
  lora_bwd_sum_body(part_dxa, ncs, nx, part_db, nrs, nb, R, scale, dxa, ld_dxa, dB,
                    ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4);
}

// The sums of mxfp8_lora_bwd_batch's jobs in one flat grid (job j: blocks first[j] .. first[j + 1] - 1).
struct LoraBwdSumBatch {
  mxfp8_lora_bwd_job job[MXFP8_LORA_BWD_MAX_JOBS];
  int first[MXFP8_LORA_BWD_MAX_JOBS + 1];
  int n, nrs, R, T;
};

__global__ __launch_bounds__(256) void lora_bwd_sum_batch_kernel(const LoraBwdSumBatch a) {
  const int b = blockIdx.x;
  int j = 0;
  while (j + 1 < a.n && a.first[j + 1] <= b) ++j;
  const mxfp8_lora_bwd_job& jb = a.job[j];
  const int64_t nx = jb.N == 128 ? 0 : (int64_t)a.T * a.R;  // one column chunk: d(xa) already written
  lora_bwd_sum_body(jb.part_dxa, (int)(jb.N / 128), nx, jb.part_db, a.nrs, jb.N * a.R, a.R, jb.scale,
                    static_cast<uint16_t*>(jb.dxa), jb.ld_dxa, jb.db,
                    ((int64_t)(b - a.first[j]) * 256 + threadIdx.x) * 4);
}

// ------------------------------------------------------------------------------------- Pᵀ · X (tn)
// The body (tn_body, tn_device.h) with its per-wave tiles in this kernel's own LDS; grid (K / 128, chunks).
template <int RP, int kD>
__global__ __launch_bounds__(256) void tn_kernel(const uint16_t* __restrict__ X, int64_t ldx,
                                                 const uint16_t* __restrict__ P, int T, int K, int chunk,
                                                 float* __restrict__ part) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[tn_lds_elems<RP>()];
  tn_body<RP, kD>(X, ldx, P, T, K, chunk, part, blockIdx.x, blockIdx.y, lds);
}

// The token reductions of mxfp8_lora_tn_batch in one flat grid (TnBatch, tn_device.h); kWide when a job has
// rank 64, so that batches of ranks 16 and 32 keep the smaller LDS footprint.
template <int kD, bool kWide>
__global__ __launch_bounds__(256) void tn_batch_kernel(const TnBatch a) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[tn_batch_lds_elems<kWide>()];
  tn_batch_block<kD, kWide>(a, blockIdx.x, lds);
}

// out = bf16(Σ_c part[c, ρ, k]) (then bf16(· scale) when scale != 1), written as [RP, K] or transposed
// [K, RP]; as fp32 holding the bf16 value (out_f32) or as bf16.  The chunks are added in order.
__device__ __forceinline__ void tn_sum_body(const float* __restrict__ part, int chunks, int RP, int K, float scale,
                                            int transpose, int out_f32, void* __restrict__ out, int64_t i) {
  const int64_t n = (int64_t)RP * K;
  if (i >= n) return;
  float v = part[i];
  int c = 1;
  for (; c + 7 < chunks; c += 8) {  // eight loads in flight, added in chunk order
    float x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = part[(int64_t)(c + u) * n + i];
#pragma unroll
    for (int u = 0; u < 8; ++u) v += x[u];
  }
  for (; c < chunks; ++c) v += part[(int64_t)c * n + i];
  v = round_bf16(v);
  if (scale != 1.0f) v = round_bf16(v * scale);
  const int64_t rho = i / K, k = i % K;
  const int64_t o = transpose ? k * RP + rho : i;
  if (out_f32) reinterpret_cast<float*>(out)[o] = v;
  else reinterpret_cast<uint16_t*>(out)[o] = bf(v);
}

__global__ __launch_bounds__(256) void tn_sum_kernel(const float* __restrict__ part, int chunks, int RP, int K,
                                                     float scale, int transpose, int out_f32, void* __restrict__ out) {
  tn_sum_body(part, chunks, RP, K, scale, transpose, out_f32, out, (int64_t)blockIdx.x * 256 + threadIdx.x);
}

// The sums of mxfp8_lora_tn_batch's jobs in one flat grid (TnSumBatch, tn_device.h).
__global__ __launch_bounds__(256) void tn_sum_batch_kernel(const TnSumBatch a) {
  const int b = blockIdx.x;
  int j = 0;
  while (j + 1 < a.n && a.first[j + 1] <= b) ++j;
  tn_sum_body(a.part[j], a.chunks, a.rp[j], a.K, a.scale[j], a.transpose[j], a.out_f32[j], a.out[j],
              (int64_t)(b - a.first[j]) * 256 + threadIdx.x);
}

// ------------------------------------------------------------------------------- backward partial sums
struct FinishArgs {
  const float *dxa_part, *dbg_part, *dbu_part, *dad_part;
  int ncg, nsb, T, N, R;
  float s_g, s_u;
  uint16_t *dxa, *xsd;        // [T, 2r] bf16 (scaled), [T, r] bf16
  float *dbg, *dbu, *dad;     // [N, r], [N, r], [r, N] fp32
};

// Four consecutive output elements per thread (16-byte loads) of dxa | xsd, dB_g, dB_u, dA_d; the partials
// are added in ascending order (fused_mlp.py:258, :319-326).
__global__ __launch_bounds__(256) void finish_kernel(FinishArgs a, int64_t total4) {
  int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total4) return;
  const int64_t R = a.R;
  int64_t n4 = (int64_t)a.T * 3 * R / 4;
  if (i < n4) {
    const float4 v = sum_ordered(reinterpret_cast<const float4*>(a.dxa_part) + i, n4, a.ncg);
    const int64_t t = (4 * i) / (3 * R), c = (4 * i) % (3 * R);  // 3R % 4 == 0: the four share row t
    const float f[4] = {v.x, v.y, v.z, v.w};
    if (c < 2 * R) {
      const float sc = c < R ? a.s_g : a.s_u;  // R % 4 == 0: the four share the scale
      const uint2 w = make_uint2(pack_bf16x2(f[0] * sc, f[1] * sc), pack_bf16x2(f[2] * sc, f[3] * sc));
      *reinterpret_cast<uint2*>(a.dxa + t * 2 * R + c) = w;
    } else {
      *reinterpret_cast<uint2*>(a.xsd + t * R + c - 2 * R) =
          make_uint2(pack_bf16x2(f[0], f[1]), pack_bf16x2(f[2], f[3]));
    }
    return;
  }
  i -= n4;
  n4 = (int64_t)a.N * R / 4;
  const float* src;
  float* dst;
  float sc;
  if (i < n4) { src = a.dbg_part; dst = a.dbg; sc = a.s_g; }
  else if (i < 2 * n4) { i -= n4; src = a.dbu_part; dst = a.dbu; sc = a.s_u; }
  else { i -= 2 * n4; src = a.dad_part; dst = a.dad; sc = 1.0f; }
  float4 v = sum_ordered(reinterpret_cast<const float4*>(src) + i, n4, a.nsb);
  if (sc != 1.0f) v = make_float4(v.x * sc, v.y * sc, v.z * sc, v.w * sc);
  reinterpret_cast<float4*>(dst)[i] = v;
}

}  // namespace

extern "C" int mxfp8_lora_prep(const float* Ag, const float* Au, const float* Bg, const float* Bu, const float* Ad,
                               const float* Bd, int64_t R, int64_t K, int64_t N, void* S, void* ST, void* bg, void* bu,
                               void* bgT, void* buT, void* ad, void* adT, void* bd, void* bdT, void* stream) {
  MX_CHECK_ARG(Ag && Au && Bg && Bu && Ad && Bd && S && ST && bg && bu && bgT && buT && ad && adT && bd && bdT,
               "mxfp8_lora_prep: null pointer");
  MX_CHECK_ARG(R > 0 && R <= 64 && K > 0 && N > 0 && K < (1 << 24) && N < (1 << 24), "mxfp8_lora_prep: bad shape");
  const int64_t total = 4 * R * K + 6 * N * R + 2 * K * R;
  PrepArgs a{Ag, Au, Bg, Bu, Ad, Bd, (uint16_t*)S, (uint16_t*)ST, (uint16_t*)bg, (uint16_t*)bu, (uint16_t*)bgT,
             (uint16_t*)buT, (uint16_t*)ad, (uint16_t*)adT, (uint16_t*)bd, (uint16_t*)bdT, (int)R, (int)K, (int)N};
  if (total < (1LL << 31) - 256) prep_kernel<int><<<(unsigned)((total + 255) / 256), 256, 0, (hipStream_t)stream>>>(a, (int)total);
  else prep_kernel<int64_t><<<(unsigned)((total + 255) / 256), 256, 0, (hipStream_t)stream>>>(a, total);
  MX_CHECK_LAUNCH("mxfp8_lora_prep");
  return MXFP8_OK;
}

namespace {

// The job table of mxfp8_pack_bf16, by value; block b of the grid works on job j where first[j] <= b < first[j + 1],
// 256 threads x 4 elements of that job (row-major over the job's rows x cols).
struct PackArgs {
  mxfp8_pack_job job[MXFP8_PACK_MAX_JOBS];
  int first[MXFP8_PACK_MAX_JOBS + 1];
  int n;
};

__global__ __launch_bounds__(256) void pack_kernel(const PackArgs a) {
  const int b = blockIdx.x;
  int j = 0;
  while (j + 1 < a.n && a.first[j + 1] <= b) ++j;
  const mxfp8_pack_job& jb = a.job[j];
  const int64_t n = jb.rows * jb.cols;
  const int64_t e0 = ((int64_t)(b - a.first[j]) * 256 + threadIdx.x) * 4;
  uint16_t* dst = static_cast<uint16_t*>(jb.dst);
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t e = e0 + u;
    if (e >= n) break;
    const int64_t r = e / jb.cols, c = e % jb.cols;
    uint16_t v = 0;
    if (jb.src) {
      v = jb.src_f32 ? (uint16_t)f32_to_bf16_bits(static_cast<const float*>(jb.src)[r * jb.src_ld + c])
                     : static_cast<const uint16_t*>(jb.src)[r * jb.src_ld + c];
    }
    dst[jb.transpose ? c * jb.dst_ld + r : r * jb.dst_ld + c] = v;
  }
}

}  // namespace

extern "C" int mxfp8_pack_bf16(const mxfp8_pack_job* jobs, int64_t n_jobs, void* stream) {
  MX_CHECK_ARG(jobs && n_jobs > 0 && n_jobs <= MXFP8_PACK_MAX_JOBS, "mxfp8_pack_bf16: need 1..%d jobs",
               MXFP8_PACK_MAX_JOBS);
  PackArgs a{};
  int64_t blocks = 0;
  for (int64_t j = 0; j < n_jobs; ++j) {
    const mxfp8_pack_job& jb = jobs[j];
    MX_CHECK_ARG(jb.dst && jb.rows >= 0 && jb.cols > 0 && jb.dst_ld >= (jb.transpose ? jb.rows : jb.cols) &&
                     (!jb.src || jb.src_ld >= jb.cols),
                 "mxfp8_pack_bf16: bad job %lld (rows=%lld cols=%lld src_ld=%lld dst_ld=%lld)", (long long)j,
                 (long long)jb.rows, (long long)jb.cols, (long long)jb.src_ld, (long long)jb.dst_ld);
    a.job[j] = jb;
    a.first[j] = (int)blocks;
    blocks += (jb.rows * jb.cols + 1023) / 1024;
    MX_CHECK_ARG(blocks < (1LL << 30), "mxfp8_pack_bf16: too large");
  }
  a.first[n_jobs] = (int)blocks;
  a.n = (int)n_jobs;
  if (blocks == 0) return MXFP8_OK;
  pack_kernel<<<(unsigned)blocks, 256, 0, (hipStream_t)stream>>>(a);
  MX_CHECK_LAUNCH("mxfp8_pack_bf16");
  return MXFP8_OK;
}

extern "C" int mxfp8_transpose_pad(const void* x, int64_t T, int64_t C, int64_t ld_x, void* out, int64_t Tpad,
                                   void* stream) {
  MX_CHECK_ARG(x && out, "mxfp8_transpose_pad: null pointer");
  MX_CHECK_ARG(T > 0 && Tpad >= T && Tpad < (1LL << 31) && (C == 16 || C == 32 || C == 64) && ld_x >= C &&
                   ld_x % 8 == 0 && mx_aligned(x, 16) && mx_aligned(out, 2),
               "mxfp8_transpose_pad: need C in {16, 32, 64}, Tpad >= T, 16-byte aligned rows of x");
  dim3 grid((unsigned)((Tpad + 255) / 256));
  hipStream_t stm = (hipStream_t)stream;
  const uint16_t* xp = (const uint16_t*)x;
  uint16_t* op = (uint16_t*)out;
  if (C == 16) transpose_pad_kernel<16><<<grid, 256, 0, stm>>>(xp, ld_x, (int)T, (int)Tpad, op);
  else if (C == 32) transpose_pad_kernel<32><<<grid, 256, 0, stm>>>(xp, ld_x, (int)T, (int)Tpad, op);
  else transpose_pad_kernel<64><<<grid, 256, 0, stm>>>(xp, ld_x, (int)T, (int)Tpad, op);
  MX_CHECK_LAUNCH("mxfp8_transpose_pad");
  return MXFP8_OK;
}

extern "C" int mxfp8_lora_nt(const void* x, int64_t T, int64_t K, int64_t ld_x, const void* w, int64_t rp, float scale,
                             void* out, void* outT, int64_t Tpad, void* stream) {
  MX_CHECK_ARG(x && w && out, "mxfp8_lora_nt: null pointer");
  MX_CHECK_ARG(T > 0 && K > 0 && K % 64 == 0 && ld_x >= K && ld_x % 8 == 0 && (rp == 16 || rp == 32 || rp == 64),
               "mxfp8_lora_nt: need K %% 64 == 0, rp in {16, 32, 64}");
  MX_CHECK_ARG(!outT || (Tpad >= T && Tpad % 32 == 0), "mxfp8_lora_nt: Tpad must be >= T and a multiple of 32");
  MX_CHECK_ARG(mx_aligned(x, 16) && mx_aligned(w, 16), "mxfp8_lora_nt: misaligned buffer");
  MX_CHECK_ARG(T < (1LL << 31) && (outT ? Tpad : T) / 32 < (1LL << 31), "mxfp8_lora_nt: too many rows");
  const int64_t rows = outT ? Tpad : (T + 31) / 32 * 32;
  dim3 grid((unsigned)(rows / 32));
  hipStream_t stm = (hipStream_t)stream;
#define NT_ARGS (const uint16_t*)x, ld_x, (const uint16_t*)w, (int)T, (int)(outT ? Tpad : 0), (int)K, scale, \
                (uint16_t*)out, (uint16_t*)outT
  if (rp == 16) nt_kernel<16><<<grid, 256, 0, stm>>>(NT_ARGS);
  else if (rp == 32) nt_kernel<32><<<grid, 256, 0, stm>>>(NT_ARGS);
  else nt_kernel<64><<<grid, 256, 0, stm>>>(NT_ARGS);
#undef NT_ARGS
  MX_CHECK_LAUNCH("mxfp8_lora_nt");
  return MXFP8_OK;
}

extern "C" int64_t mxfp8_lora_tn_chunks(int64_t T, int64_t K) {
  if (T <= 0 || K <= 0 || K % 128) return 0;
  // K / 128 column blocks x chunks of a multiple of 32 tokens.  While x fits the last-level cache (the rule
  // of lora_tn_launch), one workgroup per CU: at configuration 3 (T = 10752, K = 2048, 16 chunks) 13.7 / 16.5 us
  // for rp 16 / 32, against 14.3 / 17.1 us at 32 chunks and more for more chunks (the partials tn_sum adds grow
  // with the chunk count).  A longer x streams from HBM and needs two workgroups per CU: at configuration 4
  // (T = 142336) 111 / 136 us at 32 chunks against 182 / 236 us at 16.
  const int64_t cols = K / 128, wgs = T * K * 2 <= (192LL << 20) ? 256 : 512, want = (wgs + cols - 1) / cols;
  const int64_t blocks = (T + 31) / 32;
  const int64_t per = (blocks + want - 1) / want;
  return (blocks + per - 1) / per;
}

namespace {

// Token reduction through the caller's partial buffer `part` (chunks * rp * K floats, every used chunk's slice
// fully overwritten, so it needs no clearing): the body of mxfp8_lora_tn and mxfp8_lora_tn_noalloc.
int lora_tn_launch(const void* x, int64_t T, int64_t K, int64_t ld_x, const void* p, int64_t rp, int64_t chunks,
                   float* part, float scale, int64_t transpose, int64_t out_f32, void* out, void* stream) {
  MX_CHECK_ARG(x && p && part && out, "mxfp8_lora_tn: null pointer");
  MX_CHECK_ARG(T > 0 && K > 0 && K % 128 == 0 && ld_x >= K && ld_x % 8 == 0 && (rp == 16 || rp == 32 || rp == 64),
               "mxfp8_lora_tn: need K %% 128 == 0, rp in {16, 32, 64}");
  MX_CHECK_ARG(chunks > 0 && chunks <= 65535, "mxfp8_lora_tn: bad chunk count");
  MX_CHECK_ARG(mx_aligned(x, 16) && mx_aligned(p, 16) && mx_aligned(part, 16), "mxfp8_lora_tn: misaligned buffer");
  const int64_t blocks = (T + 31) / 32;
  const int64_t chunk = (blocks + chunks - 1) / chunks * 32;
  const int64_t used = (T + chunk - 1) / chunk;
  hipStream_t stm = (hipStream_t)stream;
  dim3 grid((unsigned)(K / 128), (unsigned)used);
#define TN_ARGS (const uint16_t*)x, ld_x, (const uint16_t*)p, (int)T, (int)K, (int)chunk, part
  // Two steps in flight per wave when x is small enough to stay in the 256 MB last-level cache after its
  // producer (configuration 3: 17.8 against 20.0 us); one when it streams from HBM, where the deeper ring
  // measured slower (x [142336, 2048]: 181 against 160 us).
  if (T * ld_x * 2 <= (192LL << 20)) {
    if (rp == 16) tn_kernel<16, 2><<<grid, 256, 0, stm>>>(TN_ARGS);
    else if (rp == 32) tn_kernel<32, 2><<<grid, 256, 0, stm>>>(TN_ARGS);
    else tn_kernel<64, 2><<<grid, 256, 0, stm>>>(TN_ARGS);
  } else {
    if (rp == 16) tn_kernel<16, 1><<<grid, 256, 0, stm>>>(TN_ARGS);
    else if (rp == 32) tn_kernel<32, 1><<<grid, 256, 0, stm>>>(TN_ARGS);
    else tn_kernel<64, 1><<<grid, 256, 0, stm>>>(TN_ARGS);
  }
#undef TN_ARGS
  MX_CHECK_LAUNCH("mxfp8_lora_tn");
  const int64_t n = rp * K;
  tn_sum_kernel<<<(unsigned)((n + 255) / 256), 256, 0, stm>>>(part, (int)used, (int)rp, (int)K, scale, (int)transpose,
                                                              (int)out_f32, out);
  MX_CHECK_LAUNCH("mxfp8_lora_tn");
  return MXFP8_OK;
}

}  // namespace

extern "C" int mxfp8_lora_tn(const void* x, int64_t T, int64_t K, int64_t ld_x, const void* p, int64_t rp,
                             int64_t chunks, float* part, float scale, int64_t transpose, int64_t out_f32, void* out,
                             void* stream) {
  return lora_tn_launch(x, T, K, ld_x, p, rp, chunks, part, scale, transpose, out_f32, out, stream);
}

namespace mxk {

int tn_batch_tables(const char* who, const mxfp8_lora_tn_job* jobs, int64_t n_jobs, int64_t T, int64_t K,
                    int64_t chunks, float* part, TnBatch& a, TnSumBatch& sa, int64_t& nb, int64_t& ns) {
  MX_CHECK_ARG(jobs && part && n_jobs >= 1 && n_jobs <= MXFP8_LORA_TN_MAX_JOBS,
               "%s: 1 to %d jobs and a partial buffer", who, MXFP8_LORA_TN_MAX_JOBS);
  MX_CHECK_ARG(T > 0 && K > 0 && K % 128 == 0 && T < (1LL << 30) && K < (1LL << 24), "%s: need K %% 128 == 0", who);
  MX_CHECK_ARG(chunks > 0 && chunks <= 65535 && mx_aligned(part, 16), "%s: bad chunks or part", who);
  const int64_t blocks = (T + 31) / 32;
  const int64_t chunk = (blocks + chunks - 1) / chunks * 32;
  const int64_t used = (T + chunk - 1) / chunk;
  a = TnBatch{};
  sa = TnSumBatch{};
  int64_t off = 0, max_ld = K;
  nb = ns = 0;
  for (int64_t j = 0; j < n_jobs; ++j) {
    const mxfp8_lora_tn_job& jb = jobs[j];
    MX_CHECK_ARG(jb.x && jb.p && jb.out && (jb.rp == 16 || jb.rp == 32 || jb.rp == 64) && jb.ld_x >= K &&
                     jb.ld_x % 8 == 0 && mx_aligned(jb.x, 16) && mx_aligned(jb.p, 16),
                 "%s: job %lld: null pointer, rp not in {16, 32, 64} or bad x stride / alignment", who, (long long)j);
    a.x[j] = (const uint16_t*)jb.x;
    a.ldx[j] = jb.ld_x;
    a.p[j] = (const uint16_t*)jb.p;
    a.rp[j] = (int)jb.rp;
    a.wide |= jb.rp == 64;
    a.part[j] = part + off;
    a.first[j] = (int)nb;
    sa.part[j] = part + off;
    sa.rp[j] = (int)jb.rp;
    sa.scale[j] = jb.scale;
    sa.transpose[j] = (int)jb.transpose;
    sa.out_f32[j] = (int)jb.out_f32;
    sa.out[j] = jb.out;
    sa.first[j] = (int)ns;
    off += used * jb.rp * K;
    nb += (K / 128) * used;
    ns += (jb.rp * K + 255) / 256;
    max_ld = std::max(max_ld, jb.ld_x);
  }
  MX_CHECK_ARG(nb < (1LL << 31), "%s: too many workgroups", who);
  a.first[n_jobs] = (int)nb;
  sa.first[n_jobs] = (int)ns;
  a.n = sa.n = (int)n_jobs;
  a.T = (int)T;
  a.K = sa.K = (int)K;
  a.chunk = (int)chunk;
  a.cols = (int)(K / 128);
  // the ring depth rule of lora_tn_launch
  a.kd = T * max_ld * 2 <= (192LL << 20) ? 2 : 1;
  sa.chunks = (int)used;
  return MXFP8_OK;
}

int tn_sum_batch_launch(const TnSumBatch& sa, int64_t ns, hipStream_t stm, const char* who) {
  tn_sum_batch_kernel<<<(unsigned)ns, 256, 0, stm>>>(sa);
  MX_CHECK_LAUNCH(who);
  return MXFP8_OK;
}

}  // namespace mxk

extern "C" int mxfp8_lora_tn_batch(const mxfp8_lora_tn_job* jobs, int64_t n_jobs, int64_t T, int64_t K,
                                   int64_t chunks, float* part, void* stream) {
  TnBatch a;
  TnSumBatch sa;
  int64_t nb = 0, ns = 0;
  const int rc = tn_batch_tables("mxfp8_lora_tn_batch", jobs, n_jobs, T, K, chunks, part, a, sa, nb, ns);
  if (rc != MXFP8_OK) return rc;
  hipStream_t stm = (hipStream_t)stream;
  if (a.kd == 2 && a.wide) tn_batch_kernel<2, true><<<(unsigned)nb, 256, 0, stm>>>(a);
  else if (a.kd == 2) tn_batch_kernel<2, false><<<(unsigned)nb, 256, 0, stm>>>(a);
  else if (a.wide) tn_batch_kernel<1, true><<<(unsigned)nb, 256, 0, stm>>>(a);
  else tn_batch_kernel<1, false><<<(unsigned)nb, 256, 0, stm>>>(a);
  MX_CHECK_LAUNCH("mxfp8_lora_tn_batch");
  return tn_sum_batch_launch(sa, ns, stm, "mxfp8_lora_tn_batch");
}

// ------------------------------------------------------------------ allocation-free token reduction
// The chunk partials of mxfp8_lora_tn_noalloc live in this file-scope device array, one copy per GPU, held until
// the process ends.  Host code never passes `scratch` itself (in host code the name is a stand-in, not a device
// address): the device address comes from hipGetSymbolAddress, looked up once per device on its first call with
// that device current, and kept in scratch_dev.  Every call on one GPU shares that GPU's array; calls that
// overlap on one GPU (different streams, or threads) race on it.
constexpr int64_t kNoAllocScratchBytes = 16LL << 20;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / 4];

namespace {

constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
float* scratch_dev[kMaxDevices] = {};

// Device address of this GPU's `scratch` (nullptr and the error message set on failure).
float* scratch_on_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    mxabi::set_error("mxfp8_lora_tn_noalloc: no current device (or device index >= %d)", kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_dev[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      mxabi::set_error("mxfp8_lora_tn_noalloc: hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                       hipGetErrorString(e));
      return nullptr;
    }
    scratch_dev[dev] = static_cast<float*>(ptr);
  }
  return scratch_dev[dev];
}

}  // namespace

extern "C" int64_t mxfp8_lora_tn_noalloc_chunks(int64_t T, int64_t K, int64_t rp) {
  if (T <= 0 || K <= 0 || K % 128 || rp <= 0) return 0;
  const int64_t fit = kNoAllocScratchBytes / 4 / (rp * K);
  return std::min(mxfp8_lora_tn_chunks(T, K), fit);
}

extern "C" int mxfp8_lora_tn_noalloc(const void* x, int64_t T, int64_t K, int64_t ld_x, const void* p, int64_t rp,
                                     float scale, int64_t transpose, int64_t out_f32, void* out, void* stream) {
  MX_CHECK_ARG(T > 0 && K > 0 && K % 128 == 0 && (rp == 16 || rp == 32 || rp == 64),
               "mxfp8_lora_tn_noalloc: need T > 0, K %% 128 == 0, rp in {16, 32, 64}");
  MX_CHECK_ARG(rp * K * 4 <= kNoAllocScratchBytes,
               "mxfp8_lora_tn_noalloc: rp * K * 4 = %lld bytes exceeds the %lld-byte static scratch",
               (long long)(rp * K * 4), (long long)kNoAllocScratchBytes);
  float* part = scratch_on_current_device();
  if (!part) return MXFP8_ERR_ARG;
  return lora_tn_launch(x, T, K, ld_x, p, rp, mxfp8_lora_tn_noalloc_chunks(T, K, rp), part, scale, transpose, out_f32,
                        out, stream);
}

extern "C" int mxfp8_mlp_bwd_finish(const float* dxa_part, const float* dbg_part, const float* dbu_part,
                                    const float* dad_part, int64_t ncg, int64_t nsb, int64_t T, int64_t N, int64_t r,
                                    float s_g, float s_u, void* dxa, void* xsd, float* dbg, float* dbu, float* dad,
                                    void* stream) {
  MX_CHECK_ARG(dxa_part && dbg_part && dbu_part && dad_part && dxa && xsd && dbg && dbu && dad,
               "mxfp8_mlp_bwd_finish: null pointer");
  MX_CHECK_ARG(ncg > 0 && nsb > 0 && T > 0 && N > 0 && (r == 16 || r == 32), "mxfp8_mlp_bwd_finish: bad shape");
  MX_CHECK_ARG(mx_aligned(dxa_part, 16) && mx_aligned(dbg_part, 16) && mx_aligned(dbu_part, 16) &&
                   mx_aligned(dad_part, 16) && mx_aligned(dxa, 8) && mx_aligned(xsd, 8) && mx_aligned(dbg, 16) &&
                   mx_aligned(dbu, 16) && mx_aligned(dad, 16),
               "mxfp8_mlp_bwd_finish: misaligned buffer");
  const int64_t total4 = (T * 3 * r + 3 * N * r) / 4;
  FinishArgs a{dxa_part, dbg_part, dbu_part, dad_part, (int)ncg, (int)nsb, (int)T, (int)N, (int)r, s_g, s_u,
               (uint16_t*)dxa, (uint16_t*)xsd, dbg, dbu, dad};
  finish_kernel<<<(unsigned)((total4 + 255) / 256), 256, 0, (hipStream_t)stream>>>(a, total4);
  MX_CHECK_LAUNCH("mxfp8_mlp_bwd_finish");
  return MXFP8_OK;
}

namespace {

int quant_lora_launch(const void* x, int64_t T, int64_t K, int64_t ld_x, void* q, void* s, const void* w, int64_t rp,
                      float scale, void* out, void* outT, int64_t Tpad, const TpJob& tp, void* stream) {
  MX_CHECK_ARG(x && q && s && w && out, "mxfp8_quant_lora: null pointer");
  MX_CHECK_ARG(T > 0 && K > 0 && K % 128 == 0 && ld_x >= K && ld_x % 8 == 0 && (rp == 16 || rp == 32 || rp == 64),
               "mxfp8_quant_lora: need K %% 128 == 0, rp in {16, 32, 64}");
  MX_CHECK_ARG(Tpad == (T + 127) / 128 * 128, "mxfp8_quant_lora: Tpad must be ceil(T / 128) * 128");
  MX_CHECK_ARG(mx_aligned(x, 16) && mx_aligned(w, 16) && mx_aligned(q, 16) && mx_aligned(s, 16),
               "mxfp8_quant_lora: misaligned buffer");
  MX_CHECK_ARG(Tpad / 32 < (1LL << 30) && T * K < (1LL << 40), "mxfp8_quant_lora: too large");
  const int64_t extra = tp.C ? (Tpad + 255) / 256 : 0;  // workgroups of the transpose job
  dim3 grid((unsigned)(Tpad / 32 + extra));
  hipStream_t stm = (hipStream_t)stream;
#define QL_ARGS (const uint16_t*)x, ld_x, (int)T, (int)K, (const uint16_t*)w, (uint8_t*)q, (uint8_t*)s, scale, \
                (uint16_t*)out, (uint16_t*)outT, (int)Tpad, tp
  if (rp == 16) quant_lora_kernel<16><<<grid, 256, 0, stm>>>(QL_ARGS);
  else if (rp == 32) quant_lora_kernel<32><<<grid, 256, 0, stm>>>(QL_ARGS);
  else quant_lora_kernel<64><<<grid, 256, 0, stm>>>(QL_ARGS);
#undef QL_ARGS
  MX_CHECK_LAUNCH("mxfp8_quant_lora");
  return MXFP8_OK;
}

}  // namespace

extern "C" int mxfp8_quant_lora(const void* x, int64_t T, int64_t K, int64_t ld_x, void* q, void* s, const void* w,
                                int64_t rp, float scale, void* out, void* outT, int64_t Tpad, void* stream) {
  return quant_lora_launch(x, T, K, ld_x, q, s, w, rp, scale, out, outT, Tpad, TpJob{nullptr, 0, 0, nullptr}, stream);
}

extern "C" int mxfp8_quant_lora_tp(const void* x, int64_t T, int64_t K, int64_t ld_x, void* q, void* s, const void* w,
                                   int64_t rp, float scale, void* out, void* outT, int64_t Tpad, const void* tx,
                                   int64_t ld_tx, int64_t tc, void* tout, void* stream) {
  MX_CHECK_ARG(tx && tout, "mxfp8_quant_lora_tp: null pointer");
  MX_CHECK_ARG((tc == 16 || tc == 32 || tc == 64) && ld_tx >= tc && ld_tx % 8 == 0 && mx_aligned(tx, 16) &&
                   mx_aligned(tout, 2),
               "mxfp8_quant_lora_tp: need tc in {16, 32, 64} and 16-byte aligned rows of tx");
  return quant_lora_launch(x, T, K, ld_x, q, s, w, rp, scale, out, outT, Tpad,
                           TpJob{(const uint16_t*)tx, ld_tx, (int)tc, (uint16_t*)tout}, stream);
}

extern "C" int mxfp8_res_lora(const void* x, const void* y, const void* xa, int64_t ld_xa, const void* b, int64_t T,
                              int64_t N, int64_t r, float scale, void* out, void* stream) {
  MX_CHECK_ARG(x && y && xa && b && out, "mxfp8_res_lora: null pointer");
  MX_CHECK_ARG(T > 0 && N > 0 && N % 128 == 0 && (r == 16 || r == 32) && ld_xa >= r,
               "mxfp8_res_lora: need N %% 128 == 0, r in {16, 32}");
  MX_CHECK_ARG(T * N < (1LL << 31), "mxfp8_res_lora: T * N must stay below 2^31");
  MX_CHECK_ARG(mx_aligned(x, 16) && mx_aligned(y, 16) && mx_aligned(b, 16) && mx_aligned(out, 16) &&
                   mx_aligned(xa, 2),
               "mxfp8_res_lora: misaligned buffer");
  const bool vec = mx_aligned(xa, 16) && ld_xa % 8 == 0;
  dim3 grid((unsigned)((T + 31) / 32), (unsigned)(N / 128));
  hipStream_t stm = (hipStream_t)stream;
#define RL_ARGS (const uint16_t*)x, (const uint16_t*)y, (const uint16_t*)xa, ld_xa, (const uint16_t*)b, (int)T, (int)N, \
                scale, (uint16_t*)out
  if (r == 16) {
    if (vec) res_lora_kernel<16, true><<<grid, 256, 0, stm>>>(RL_ARGS);
    else res_lora_kernel<16, false><<<grid, 256, 0, stm>>>(RL_ARGS);
  } else {
    if (vec) res_lora_kernel<32, true><<<grid, 256, 0, stm>>>(RL_ARGS);
    else res_lora_kernel<32, false><<<grid, 256, 0, stm>>>(RL_ARGS);
  }
#undef RL_ARGS
  MX_CHECK_LAUNCH("mxfp8_res_lora");
  return MXFP8_OK;
}

// Row chunks for at most `target` workgroups over (chunks, N / 128), the workgroups the CUs hold at once (two per
// CU with the LoRA products, whose dB partials grow with the chunk count; three for the codes alone), so the grid
// runs in one round.  Rounding the chunk count up instead gave dy [10752, 6144] 11 x 48 = 528 workgroups, a second
// round of 16 for the 512 slots: 58.3 against 52.2 us for 8 x 48 (graph timing, one box).
static int64_t lora_bwd_rows(int64_t T, int64_t N, int64_t target) {
  if (T <= 0 || N <= 0 || N % 128) return 0;
  const int64_t blocks = (T + 127) / 128 * 4;  // 32-row blocks up to the padded end of the last 128-row tile
  const int64_t cs = N / 128, want = std::max<int64_t>(1, target / cs);
  const int64_t per = (blocks + std::min(want, blocks) - 1) / std::min(want, blocks);
  return (blocks + per - 1) / per;
}

extern "C" int64_t mxfp8_lora_bwd_chunks(int64_t T, int64_t N) { return lora_bwd_rows(T, N, 512); }

extern "C" int mxfp8_lora_bwd(const void* dy, int64_t T, int64_t N, int64_t ld_dy, void* q, int64_t ld_q, void* s,
                              int64_t s_col_tiles, int64_t col_tile_off, const void* xa, int64_t ld_xa, const void* b,
                              int64_t r, float scale, void* dxa, int64_t ld_dxa, float* db, float* part_dxa,
                              float* part_db, void* stream) {
  const bool quant = q != nullptr, lora = xa != nullptr;
  MX_CHECK_ARG(dy && (quant || lora), "mxfp8_lora_bwd: need dy and q/s or xa");
  MX_CHECK_ARG(T > 0 && N > 0 && N % 128 == 0 && ld_dy >= N && ld_dy % 8 == 0 && T * ld_dy < (1LL << 40),
               "mxfp8_lora_bwd: need N %% 128 == 0");
  MX_CHECK_ARG(!quant || (s && ld_q % 16 == 0 && col_tile_off >= 0 && col_tile_off * 128 + N <= ld_q &&
                          col_tile_off * 128 + N <= s_col_tiles * 128 && mx_aligned(q, 16) && mx_aligned(s, 4)),
               "mxfp8_lora_bwd: bad code / scale destination");
  MX_CHECK_ARG(!lora || (b && dxa && db && part_dxa && part_db && (r == 16 || r == 32) && ld_xa >= r &&
                         ld_xa % 8 == 0 && ld_dxa >= r && mx_aligned(xa, 16) && mx_aligned(b, 2)),
               "mxfp8_lora_bwd: LoRA needs xa, B, dxa, dB and partial buffers, r in {16, 32}");
  MX_CHECK_ARG(mx_aligned(dy, 16), "mxfp8_lora_bwd: misaligned dy");
  const int64_t rs = lora ? mxfp8_lora_bwd_chunks(T, N) : lora_bwd_rows(T, N, 768);
  const int64_t Tpad = (T + 127) / 128 * 128, blocks = Tpad / 32;
  const int64_t chunk = (blocks + rs - 1) / rs * 32;
  const int64_t used = (Tpad + chunk - 1) / chunk;
  hipStream_t stm = (hipStream_t)stream;
  dim3 grid((unsigned)used, (unsigned)(N / 128));
#define LB_ARGS (const uint16_t*)dy, ld_dy, (int)T, (int)N, (int)Tpad, (int)chunk, (uint8_t*)q, ld_q, (uint8_t*)s, \
                s_col_tiles, (int)col_tile_off, (const uint16_t*)xa, ld_xa, (const uint16_t*)b, part_dxa, part_db,     \
                (uint16_t*)dxa, ld_dxa, scale
  if (!lora) lora_bwd_kernel<16, true, false><<<grid, 256, 0, stm>>>(LB_ARGS);
  else if (r == 16) {
    if (quant) lora_bwd_kernel<16, true, true><<<grid, 256, 0, stm>>>(LB_ARGS);
    else lora_bwd_kernel<16, false, true><<<grid, 256, 0, stm>>>(LB_ARGS);
  } else {
    if (quant) lora_bwd_kernel<32, true, true><<<grid, 256, 0, stm>>>(LB_ARGS);
    else lora_bwd_kernel<32, false, true><<<grid, 256, 0, stm>>>(LB_ARGS);
  }
#undef LB_ARGS
  MX_CHECK_LAUNCH("mxfp8_lora_bwd");
  if (lora) {
    const int64_t nx = N == 128 ? 0 : T * r, total = nx + N * r;  // one column chunk: d(xa) already written
    lora_bwd_sum_kernel<<<(unsigned)((total / 4 + 255) / 256), 256, 0, stm>>>(
        part_dxa, (int)(N / 128), nx, part_db, (int)used, N * r, (int)r, scale, (uint16_t*)dxa, ld_dxa, db);
    MX_CHECK_LAUNCH("mxfp8_lora_bwd");
  }
  return MXFP8_OK;
}

extern "C" int64_t mxfp8_lora_bwd_batch_chunks(int64_t T, int64_t n_total) { return lora_bwd_rows(T, n_total, 512); }

extern "C" int mxfp8_lora_bwd_batch(const mxfp8_lora_bwd_job* jobs, int64_t n_jobs, int64_t T, int64_t r, void* q,
                                    int64_t ld_q, void* s, int64_t s_col_tiles, void* stream) {
  MX_CHECK_ARG(jobs && n_jobs > 0 && n_jobs <= MXFP8_LORA_BWD_MAX_JOBS && T > 0 && (r == 16 || r == 32),
               "mxfp8_lora_bwd_batch: need 1..%d jobs, T > 0, r in {16, 32}", MXFP8_LORA_BWD_MAX_JOBS);
  const bool quant = q != nullptr;
  MX_CHECK_ARG(!quant || (s && ld_q % 16 == 0 && mx_aligned(q, 16) && mx_aligned(s, 4)),
               "mxfp8_lora_bwd_batch: bad code / scale destination");
  int64_t n_total = 0;
  for (int64_t j = 0; j < n_jobs; ++j) {
    const mxfp8_lora_bwd_job& jb = jobs[j];
    MX_CHECK_ARG(jb.dy && jb.N > 0 && jb.N % 128 == 0 && jb.ld_dy >= jb.N && jb.ld_dy % 8 == 0 &&
                     T * jb.ld_dy < (1LL << 40) && mx_aligned(jb.dy, 16),
                 "mxfp8_lora_bwd_batch: job %lld: need N %% 128 == 0 and 16-byte aligned dy rows", (long long)j);
    MX_CHECK_ARG(!quant || (jb.col_tile_off >= 0 && jb.col_tile_off * 128 + jb.N <= ld_q &&
                            jb.col_tile_off * 128 + jb.N <= s_col_tiles * 128),
                 "mxfp8_lora_bwd_batch: job %lld: bad code / scale destination", (long long)j);
    MX_CHECK_ARG(jb.xa && jb.b && jb.dxa && jb.db && jb.part_dxa && jb.part_db && jb.ld_xa >= r && jb.ld_xa % 8 == 0 &&
                     jb.ld_dxa >= r && mx_aligned(jb.xa, 16) && mx_aligned(jb.b, 2),
                 "mxfp8_lora_bwd_batch: job %lld: needs xa, B, dxa, dB and partial buffers", (long long)j);
    n_total += jb.N;
  }
  const int64_t rs = mxfp8_lora_bwd_batch_chunks(T, n_total);
  const int64_t Tpad = (T + 127) / 128 * 128, blocks = Tpad / 32;
  const int64_t chunk = (blocks + rs - 1) / rs * 32;
  const int64_t used = (Tpad + chunk - 1) / chunk;
  LoraBwdBatch a{};
  LoraBwdSumBatch b{};
  int64_t wgs = 0, sum_blocks = 0;
  for (int64_t j = 0; j < n_jobs; ++j) {
    a.job[j] = b.job[j] = jobs[j];
    a.first[j] = (int)wgs;
    b.first[j] = (int)sum_blocks;
    wgs += used * (jobs[j].N / 128);
    const int64_t total = (jobs[j].N == 128 ? 0 : T * r) + jobs[j].N * r;
    sum_blocks += (total / 4 + 255) / 256;
  }
  MX_CHECK_ARG(wgs < (1LL << 31) && sum_blocks < (1LL << 31), "mxfp8_lora_bwd_batch: too large");
  a.first[n_jobs] = (int)wgs;
  b.first[n_jobs] = (int)sum_blocks;
  a.n = b.n = (int)n_jobs;
  a.T = b.T = (int)T;
  a.Tpad = (int)Tpad;
  a.chunk = (int)chunk;
  a.used = (int)used;
  a.q = (uint8_t*)q;
  a.ld_q = ld_q;
  a.s = (uint8_t*)s;
  a.s_col_tiles = s_col_tiles;
  b.nrs = (int)used;
  b.R = (int)r;
  hipStream_t stm = (hipStream_t)stream;
  if (r == 16) {
    if (quant) lora_bwd_batch_kernel<16, true><<<(unsigned)wgs, 256, 0, stm>>>(a);
    else lora_bwd_batch_kernel<16, false><<<(unsigned)wgs, 256, 0, stm>>>(a);
  } else {
    if (quant) lora_bwd_batch_kernel<32, true><<<(unsigned)wgs, 256, 0, stm>>>(a);
    else lora_bwd_batch_kernel<32, false><<<(unsigned)wgs, 256, 0, stm>>>(a);
  }
  MX_CHECK_LAUNCH("mxfp8_lora_bwd_batch");
  lora_bwd_sum_batch_kernel<<<(unsigned)sum_blocks, 256, 0, stm>>>(b);
  MX_CHECK_LAUNCH("mxfp8_lora_bwd_batch");
  return MXFP8_OK;
}
