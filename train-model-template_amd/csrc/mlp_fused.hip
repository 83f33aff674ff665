// Fused SwiGLU / LoRA / MX-requantization kernels of the MXFP8 MLP for gfx950 (forward and backward), and the
// fixed-order partial-sum reduction they feed.
//
// Reference math (every bf16 rounding point kept):
//   forward  /root/reference/scripts/fused_mlp.py:65-109 (_gu_tile, _fwd_kernel), wrapper :198-215 (mlp_fwd)
//     g = bf16(gu[:, j] + s_g * xs_g·bgᵀ), u = bf16(gu[:, N + j] + s_u * xs_u·buᵀ)
//     h = bf16(g / (exp(-g) + 1) * u);  MX(h) -> q_h, s_h;  xS_down partial = h · adᵀ
//   backward /root/reference/scripts/fused_mlp.py:112-175 (_bwd_kernel), wrapper :218-259 (mlp_bwd)
//     recompute g, u, silu, h;  dh = bf16(dhm + dxd · ad);  du = bf16(dh * silu)
//     sig = sigmoid(g);  dg = bf16(dh * u * sig * (g * (1 - sig) + 1))
//     MX([dg | du]) into one [T, 2N] buffer;  partials of dB_g = dgᵀ·xs_g, dB_u = duᵀ·xs_u, dA_dᵀ = hᵀ·dxd,
//     dxa_g = dg·bg, dxa_u = du·bu, xS_down = h·adᵀ
// Partial sums are reduced in a fixed order (no atomics), as the reference does with .sum(0).
//
// Register layout of an element tile: a 32 x 32 (row m, column j) tile in the 32x32 accumulator layout, lane
// l owning row m = l % 32 and columns j = (i/4)*8 + (l/32)*4 + i%4 of register i.  That is the layout of
// D = mfma_32x32x16_bf16(A = weight rows j, B = activation rows m), so the rank-r LoRA products land in the
// registers of the elements they update.  For products that reduce over j, the element registers
// themselves are the B operand: the instruction sums over its k index in any order, so taking k-step s as
// registers 8s..8s+7 (columns {(i/4)*8 + (l/32)*4 + i%4}) only requires the A operand (a [r, N] matrix row
// per lane) to be read in the same column order.  Products that reduce over m transpose the bf16 tile
// through LDS.
#include <type_traits>

#include "abi_common.h"
#include "mx_device.h"

using namespace mxk;

namespace {

__device__ __forceinline__ int tile_col(int i, int lane) { return (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3); }

// registers 8s..8s+7 of an element tile held as packed words w[4s..4s+3], as an MFMA operand
__device__ __forceinline__ v8bf words_bf8(const uint32_t* w) { return as_bf8(make_uint4(w[0], w[1], w[2], w[3])); }

// ---------------------------------------------------------------------------------------------- forward
// Column order of the forward tiles.  The LoRA-B product D[a][m] = Σ_ρ W[j(a), ρ] X[m, ρ] may take any weight
// row for MFMA row a; choosing j(a) = pi_col(a) puts, in lane l, the 16 CONTIGUOUS columns lg*16 + i
// (i = register, lg = l / 32) of row m = l % 32.  A lane then loads its gate / up values as two 16-byte
// pieces, quantizes 16 adjacent codes of one 32-block with its partner lane l ^ 32, and stores them as one
// 16-byte word (the accumulator order of the previous tile layout needed four 8-byte loads and four 4-byte
// stores per 16 values).
// Grid (ceil(Tpad / 128), column groups): wave w of workgroup b owns the 32-row block 4b + w and walks every
// 32-column tile of the group, loading tile t + 1 while it computes tile t; the four waves of a workgroup
// walk the same tiles, so they share the LoRA weight rows in L1.  A wave sums its own xS_down partial over the
// group's columns in registers and stores it, so no wave ever waits for another.  Rows past T compute row
// T - 1 again and store the same bytes there (every store is unconditional, so the compiler's memory-counter
// waits stay exact); only their scale bytes differ (0 in the padded rows of the last scale tile).
// Tiles in flight per wave (1 or 2) and the register budget that goes with it: two tiles ahead at 2 waves per
// SIMD (180 VGPRs) measured ~10 us per step faster than one tile ahead at 3 (148 VGPRs), on one box, twice.
#ifndef MX_FWD_AHEAD
#define MX_FWD_AHEAD 2
#endif
#ifndef MX_FWD_WAVES_PER_SIMD
#define MX_FWD_WAVES_PER_SIMD 2
#endif
constexpr int kFwdWavesPerSimd = MX_FWD_WAVES_PER_SIMD;  // register budget 512 / n VGPRs (n = 4 spills: measured slower)
template <int R, bool kWriteQ, bool kH>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kFwdWavesPerSimd, 8))) void fwd_kernel(
    const uint16_t* __restrict__ gu, const uint16_t* __restrict__ xs, const uint16_t* __restrict__ bg,
    const uint16_t* __restrict__ bu, const uint16_t* __restrict__ ad, int T, int Tpad, int N, int tiles_per_group,
    float s_g, float s_u, uint8_t* __restrict__ q, uint8_t* __restrict__ s, float* __restrict__ part,
    uint16_t* __restrict__ h_out, bool q_tiled, bool gu_ft) {
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lg = lane >> 5;
  const int rb = blockIdx.x * 4 + w;
  if (rb * 32 >= Tpad) return;  // wave-uniform
  const int m = rb * 32 + (lane & 31);
  const bool live = m < T;
  const int mc = live ? m : T - 1;
  v8bf xg[R / 16], xu[R / 16];
#pragma unroll
  for (int h = 0; h < R / 16; ++h) {
    xg[h] = load_bf8(xs + (int64_t)mc * 2 * R + h * 16 + lg * 8);
    xu[h] = load_bf8(xs + (int64_t)mc * 2 * R + R + h * 16 + lg * 8);
  }
  const int rho = lane & 31;
  const uint16_t* adrow = ad + (int64_t)(rho < R ? rho : 0) * N + lg * 16;
  v16f acc = v16f{};  // xS_down partial D[ρ][m]
  const int t0 = blockIdx.y * tiles_per_group, t_end = t0 + tiles_per_group;
  // Every operand of a tile is loaded one tile ahead, together: the memory counter completes in order, so a
  // load issued after the prefetch and used in the same tile would wait for the prefetch as well.
  struct TileIn {
    uint32_t g[8], u[8];          // gate / up values of the lane's 16 columns
    v8bf bg[R / 16], bu[R / 16];  // LoRA-B weight rows jb + pi_col(lane % 32)
    v8bf ad[2];                   // ad[ρ, jb + lg*16 + 8 ks + 0..7], ρ = lane % 32 (zero past r)
  };
  auto fetch = [&](int t, TileIn& in) {
    const int jb = t * 32;
    load16_rc(gu, mc, jb + lg * 16, 2 * N, gu_ft, in.g);  // this lane's 16 columns of the tile
    load16_rc(gu, mc, N + jb + lg * 16, 2 * N, gu_ft, in.u);
    const int64_t wr = (int64_t)(jb + pi_col(lane & 31)) * R + lg * 8;
#pragma unroll
    for (int h = 0; h < R / 16; ++h) {
      in.bg[h] = load_bf8(bg + wr + h * 16);
      in.bu[h] = load_bf8(bu + wr + h * 16);
    }
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {  // load, then select: a branch here would blur the counter waits
      const v8bf v = load_bf8(adrow + jb + 8 * ks);
      in.ad[ks] = rho < R ? v : v8bf{};
    }
  };
  // one tile: compute from `cur` while `nxt` (tile t + 1) is in flight
  auto tile = [&](int t, const TileIn& cur, TileIn& nxt) {
    const int jb = t * 32;
    fetch(min(t + MX_FWD_AHEAD, t_end - 1), nxt);  // past the group's end this reloads a tile, unused
    __builtin_amdgcn_sched_barrier(0);  // issue the prefetch here, a whole tile before its use
    // g and u as packed bf16 pairs, one at a time (each rank-r product is live only while it is added)
    uint32_t gp[8], hw[8];  // hw: first u, then h, as packed bf16 pairs (columns lg*16 + i, i + 1)
    {
      const v16f d = lora_pi<R>(cur.bg, xg);
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        float g0 = bf16_lo(cur.g[i / 2]) + s_g * d[i], g1 = bf16_hi(cur.g[i / 2]) + s_g * d[i + 1];
        gp[i / 2] = rnd2(g0, g1);
      }
    }
    {
      const v16f d = lora_pi<R>(cur.bu, xu);
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        float u0 = bf16_lo(cur.u[i / 2]) + s_u * d[i], u1 = bf16_hi(cur.u[i / 2]) + s_u * d[i + 1];
        hw[i / 2] = rnd2(u0, u1);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float g0 = bf16_lo(gp[i]), g1 = bf16_hi(gp[i]);
      float h0 = (g0 * fast_sigmoid(g0)) * bf16_lo(hw[i]), h1 = (g1 * fast_sigmoid(g1)) * bf16_hi(hw[i]);
      hw[i] = rnd2(h0, h1);
    }
    if (kWriteQ) quant16(hw, lane, m, live, q, mc, N, q_tiled, jb + lg * 16, s, N / 128);
    if (kH) {
      uint4* o = reinterpret_cast<uint4*>(h_out + (int64_t)mc * N + jb + lg * 16);
      o[0] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
      o[1] = make_uint4(hw[4], hw[5], hw[6], hw[7]);
    }
    // xS_down: D[ρ][m] += Σ_j ad[ρ, j] h[m, j]; MFMA k step ks covers, in lane l, columns lg*16 + 8 ks + 0..7
    // (registers 4ks..4ks+3 of hw), and the A operand row ρ = lane % 32 holds ad at the same columns
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cur.ad[ks], words_bf8(hw + 4 * ks), acc, 0, 0, 0);
  };
#if MX_FWD_AHEAD == 2
  TileIn b0, b1, b2;  // rotating buffers, two tiles in flight: tile t computes from one, t + 2 loads into another
  fetch(t0, b0);
  fetch(min(t0 + 1, t_end - 1), b1);
  int t = t0;
  for (; t + 2 < t_end; t += 3) {
    tile(t, b0, b2);
    tile(t + 1, b1, b0);
    tile(t + 2, b2, b1);
  }
  if (t < t_end) tile(t, b0, b2);
  if (t + 1 < t_end) tile(t + 1, b1, b0);
#else
  TileIn b0, b1;  // alternating buffers: no register copies between tiles
  fetch(t0, b0);
  int t = t0;
  for (; t + 1 < t_end; t += 2) {
    tile(t, b0, b1);
    tile(t + 1, b1, b0);
  }
  if (t < t_end) tile(t, b0, b1);
#endif
  // acc lane l: m = l % 32, ρ = (i/4)*8 + (l/32)*4 + i%4
  if (live) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int rr = tile_col(i, lane);
      if (rr < R) part[((int64_t)blockIdx.y * T + m) * R + rr] = acc[i];
    }
  }
}

// --------------------------------------------------------------------------------------------- backward
// Grid (super-blocks of SB rows, column groups of CG columns), 256 threads = 4 waves.  The workgroup walks its
// column group in quads of 128 columns (wave w on tile 4q + w) and, inside a quad, its super-block in 32-row
// blocks, in the forward kernel's column order (lane l: row m = l % 32, columns lg*16 + 0..15 of the tile).
//   per tile: recompute g, u, h; dh = bf16(dhm + dxd·ad); du, dg; MX(dg), MX(du) (codes + scales);
//     dxa_g | dxa_u | xS_down products D[ρ][m] over the tile's columns (MFMA, k = columns), summed over the
//     quad's 4 waves in LDS (fixed order) and stored (first quad) or added (later quads) into the column
//     group's [T, 3r] partial;
//     dB_g, dB_u, dA_dᵀ contributions D[j][ρ] (16x16x32 MFMA, k = rows): the wave writes its dg, then du,
//     then h rows to its LDS tile and reads each back column-wise with ds_read_b64_tr_b16; accumulated over
//     the super-block in registers and stored after it.
// The large operands of the next row block (gu, dhm) are loaded one row block ahead.  The small per-row operands
// (xs, dxd and their transposed copies, L2-resident; the same 6 KB at r = 16 for every wave of the workgroup):
//   r = 16 (kStage): staged in LDS one row block ahead, by global_load_lds DMAs issued at the start of the row
//     block before (each 1 KB DMA lands as the lane-ordered MFMA operand, so the reads are conflict-free
//     ds_read_b128), one copy per workgroup instead of one per wave.  Each wave drains its memory counter before
//     the row block's barrier, and the block's code, scale and partial stores are issued after that barrier:
//     the memory counter completes in issue order, so a wait for a load issued behind a store also waits for
//     the store, and the previous form's first wait of every row block (for the small loads, issued behind the
//     previous block's stores) paid the stores' latency.  Configuration 3, graph timing, two alternating pairs
//     on one box, outputs bit-identical: 148.1-149.6 against 140.8-144.4 us;
//   r = 32: loaded per wave at the start of each row block, before the next block's large operands, so
//     waiting for them leaves the prefetch in flight (the staged form's 24 KB would lower the 4-wave kernel's
//     workgroups per CU).
// Rows past T quantize row T - 1 again (the same bytes) and then zero their values, so they add nothing to
// dB / dA_d.
// Register budget: two waves per SIMD (<= 256 VGPRs; with three the kernel spills), i.e. two workgroups per
// CU (58 KB of LDS each at r = 16).
// kQ = 2: 8 waves, two quads side by side (wave w on tile 8o + w of the column group): the dxa products are
// summed over all 8 waves in LDS, so there is one partial per 256 columns instead of per 128 (half the partial
// bytes written here and read by the finish); one workgroup per CU (116 KB of LDS at r = 16), still two waves
// per SIMD.  With two product buffers (r = 16) one barrier per row block replaces two: 1-4% faster alone
// (151.9-154.7 against 148.9-152.4 us at configuration 3, three alternating pairs on one box, bit-identical).
// gu is read once here, with non-temporal loads, so it does not push dhm (written by the GEMM just before) and
// the MX(dg | du) codes out of the last-level cache (with the gate|up epilogue's non-temporal gu stores, MX_NT_GU
// in mx_gemm.hip: 10-17 us per configuration-3 step faster over five A/B pairs on one box).
#ifndef MX_BWD_NT_LOAD
#define MX_BWD_NT_LOAD 1
#endif
template <int R, bool kQuant, bool kDgu, int kQ = 1>
__global__ __launch_bounds__(256 * kQ) __attribute__((amdgpu_waves_per_eu(2, 8))) void bwd_kernel(
    const uint16_t* __restrict__ gu, const uint16_t* __restrict__ xs, const uint16_t* __restrict__ xsT,
    const uint16_t* __restrict__ dhm, const uint16_t* __restrict__ dxd, const uint16_t* __restrict__ dxdT,
    const uint16_t* __restrict__ bg, const uint16_t* __restrict__ bu, const uint16_t* __restrict__ bgT,
    const uint16_t* __restrict__ buT, const uint16_t* __restrict__ ad, const uint16_t* __restrict__ adT, int T,
    int Tpad, int N, int SB, int CG, float s_g, float s_u, uint8_t* __restrict__ q, uint8_t* __restrict__ s,
    float* __restrict__ dxa_part, float* __restrict__ dbg_part, float* __restrict__ dbu_part,
    float* __restrict__ dad_part, uint16_t* __restrict__ dgu_out, bool q_tiled, bool gu_ft) {
  constexpr int kW = 4 * kQ, kCols = 128 * kQ;  // waves, columns per pass over the column group
  // kRB buffers of the per-wave products: with two, row block b fills buffer b % 2 while the waves still sum
  // block b - 1's, so one barrier per row block suffices; taken where they fit the LDS of the workgroups a CU
  // holds now (one with 8 waves, two with 4)
  constexpr bool kStage = R == 16;                                      // small operands staged in LDS
  constexpr int kOps = 6 * (R / 16), kOpDma = (kOps + kW - 1) / kW;  // 1 KB operand images, DMAs per wave
  constexpr int kRedBytes = kW * 32 * (3 * R + 1) * 4, kTrBytes = kW * 32 * kTrLd * 2;
  constexpr int kStageBytes = kStage ? 2 * kOps * 1024 : 0, kLdsCap = (kQ == 2 ? 160 : 80) * 1024;
  constexpr int kRB = 2 * kRedBytes + kTrBytes + kStageBytes <= kLdsCap ? 2 : 1;
  static_assert(kRB * kRedBytes + kTrBytes + kStageBytes <= kLdsCap, "LDS of the workgroups a CU holds");
  __shared__ float red[kRB][kW][32][3 * R + 1];                        // per-wave dxa | dxa_u | xS products
  __shared__ __attribute__((aligned(16))) uint16_t trt[kW][32 * kTrLd];  // per-wave dg, then du, then h rows
  // two row blocks' small operands: images xg, xu, xd, tg, tu, td (R / 16 each), lane l's 16 bytes at 16 l
  __shared__ __attribute__((aligned(16))) uint8_t sop[kStage ? 2 : 1][kStage ? kOps : 1][kStage ? 1024 : 16];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lg = lane >> 5;
  const int r0 = blockIdx.x * SB, r1 = min(r0 + SB, Tpad);
  const int c0 = blockIdx.y * CG;
  const int rho = lane & 31;
  const int rho_c = rho < R ? rho : 0;
  struct RowIn {
    uint32_t g[8], u[8], d[8];  // gate, up, dhm of the lane's row and 16 columns
  };
  for (int oc = 0; oc < CG / kCols; ++oc) {
    const int jb = c0 + oc * kCols + w * 32;  // this wave's tile
    // weights of this tile: LoRA-B rows jb + pi_col(lane % 32) (bg, bu, adᵀ) and, for the products that
    // reduce over the columns, rows ρ of bgᵀ, buᵀ, ad at the lane's columns
    v8bf wbg[R / 16], wbu[R / 16], wad[R / 16], fbg[2], fbu[2], fad[2];
    {
      const int64_t wr = (int64_t)(jb + pi_col(lane & 31)) * R + lg * 8;
#pragma unroll
      for (int h = 0; h < R / 16; ++h) {
        wbg[h] = load_bf8(bg + wr + h * 16);
        wbu[h] = load_bf8(bu + wr + h * 16);
        wad[h] = load_bf8(adT + wr + h * 16);
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {  // load, then select (no branch)
        const int64_t off = (int64_t)rho_c * N + jb + lg * 16 + 8 * ks;
        const v8bf a = load_bf8(bgT + off), b = load_bf8(buT + off), c = load_bf8(ad + off);
        fbg[ks] = rho < R ? a : v8bf{};
        fbu[ks] = rho < R ? b : v8bf{};
        fad[ks] = rho < R ? c : v8bf{};
      }
    }
    // dB_g, dB_u, dA_d of this tile as D[j][ρ]: lane l holds ρ = 16 h + l % 16, j = jb + 16 jh + (l/16)*4 + i
    v4f dbg[2][R / 16], dbu[2][R / 16], dad[2][R / 16];
#pragma unroll
    for (int jh = 0; jh < 2; ++jh)
#pragma unroll
      for (int h = 0; h < R / 16; ++h) dbg[jh][h] = dbu[jh][h] = dad[jh][h] = v4f{};
    auto fetch = [&](int rb, RowIn& in) {
      const int mc = min(rb + (lane & 31), T - 1);
#if MX_BWD_NT_LOAD
      load16_rc_nt(gu, mc, jb + lg * 16, 2 * N, gu_ft, in.g);
      load16_rc_nt(gu, mc, N + jb + lg * 16, 2 * N, gu_ft, in.u);
#else
      load16_rc(gu, mc, jb + lg * 16, 2 * N, gu_ft, in.g);
      load16_rc(gu, mc, N + jb + lg * 16, 2 * N, gu_ft, in.u);
#endif
      load16_rc(dhm, mc, jb + lg * 16, N, gu_ft, in.d);
    };
    // DMA of row block rbn's small operands into sop[sb]: wave w issues images w * kOpDma + j (modulo kOps: the
    // slots past the last image repeat one, the same bytes to the same place), so every wave issues kOpDma DMAs
    // and one memory-counter wait fits all.  Lane l fetches exactly the 16 bytes that it reads back as its MFMA
    // operand (the per-wave loads of the r = 32 form below): xs / dxd rows min(rbn + l % 32, T - 1), xsᵀ / dxdᵀ
    // rows 16 h + l % 16 at columns rbn + 8 (l / 16) (rbn + 32 <= Tpad, the padded width).
    auto stage = [&](int rbn, int sb) {
#pragma unroll
      for (int j = 0; j < kOpDma; ++j) {
        const int o = (w * kOpDma + j) % kOps, kind = o / (R / 16), h = o % (R / 16);
        const int mcn = min(rbn + (lane & 31), T - 1);
        const int rr = h * 16 + (lane & 15), mo = rbn + (lane >> 4) * 8;
        const uint16_t* src;
        if (kind == 0) src = xs + (int64_t)mcn * 2 * R + h * 16 + lg * 8;
        else if (kind == 1) src = xs + (int64_t)mcn * 2 * R + R + h * 16 + lg * 8;
        else if (kind == 2) src = dxd + (int64_t)mcn * R + h * 16 + lg * 8;
        else if (kind == 3) src = xsT + (int64_t)rr * Tpad + mo;
        else if (kind == 4) src = xsT + (int64_t)(R + rr) * Tpad + mo;
        else src = dxdT + (int64_t)rr * Tpad + mo;
        dma16(src, lds_addr(&sop[sb][o][0]));
      }
    };
    auto sop_read = [&](int sb, int o) { return as_bf8(*reinterpret_cast<const uint4*>(&sop[sb][o][lane * 16])); };
    auto block = [&](int rb, const RowIn& cur, RowIn& nxt, const int buf) {
      const int m = rb + (lane & 31);
      const bool live = m < T;
      const int mc = live ? m : T - 1;
      const int sb = ((rb - r0) >> 5) & 1;  // staged operands of this row block (kStage)
      // small operands of this row block first (see above), then the next row block's large ones
      v8bf xg[R / 16], xu[R / 16], xd[R / 16], tg[R / 16], tu[R / 16], td[R / 16];
      if constexpr (kStage) {
        // the next row block's DMA goes to the other buffer, which the waves finished reading before the
        // previous row block's barrier
        stage(min(rb + 32, r1 - 32), sb ^ 1);
#pragma unroll
        for (int h = 0; h < R / 16; ++h) {
          xg[h] = sop_read(sb, 0 * (R / 16) + h);
          xu[h] = sop_read(sb, 1 * (R / 16) + h);
          xd[h] = sop_read(sb, 2 * (R / 16) + h);
        }
      } else {
#pragma unroll
        for (int h = 0; h < R / 16; ++h) {
          xg[h] = load_bf8(xs + (int64_t)mc * 2 * R + h * 16 + lg * 8);
          xu[h] = load_bf8(xs + (int64_t)mc * 2 * R + R + h * 16 + lg * 8);
          xd[h] = load_bf8(dxd + (int64_t)mc * R + h * 16 + lg * 8);
          const int rr = h * 16 + (lane & 15), mo = rb + (lane >> 4) * 8;
          tg[h] = load_bf8(xsT + (int64_t)rr * Tpad + mo);
          tu[h] = load_bf8(xsT + (int64_t)(R + rr) * Tpad + mo);
          td[h] = load_bf8(dxdT + (int64_t)rr * Tpad + mo);
        }
      }
      fetch(min(rb + 32, r1 - 32), nxt);  // past the super-block's end this reloads a row block, unused
      __builtin_amdgcn_sched_barrier(0);
      // g, u, dh as packed bf16 pairs, one rank-r product at a time
      uint32_t gp[8], upk[8], dp[8];
      {
        const v16f d = lora_pi<R>(wbg, xg);
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
          float a = bf16_lo(cur.g[i / 2]) + s_g * d[i], b = bf16_hi(cur.g[i / 2]) + s_g * d[i + 1];
          gp[i / 2] = rnd2(a, b);
        }
      }
      {
        const v16f d = lora_pi<R>(wbu, xu);
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
          float a = bf16_lo(cur.u[i / 2]) + s_u * d[i], b = bf16_hi(cur.u[i / 2]) + s_u * d[i + 1];
          upk[i / 2] = rnd2(a, b);
        }
      }
      {
        const v16f d = lora_pi<R>(wad, xd);
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
          float a = bf16_lo(cur.d[i / 2]) + d[i], b = bf16_hi(cur.d[i / 2]) + d[i + 1];
          dp[i / 2] = rnd2(a, b);  // dh
        }
      }
      uint32_t dgw[8], duw[8], hw[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float g0 = bf16_lo(gp[i]), g1 = bf16_hi(gp[i]);
        const float u0 = bf16_lo(upk[i]), u1 = bf16_hi(upk[i]);
        const float d0 = bf16_lo(dp[i]), d1 = bf16_hi(dp[i]);
        const float sg0 = fast_sigmoid(g0), sg1 = fast_sigmoid(g1);
        const float sl0 = g0 * sg0, sl1 = g1 * sg1;
        float h0 = sl0 * u0, h1 = sl1 * u1;
        hw[i] = rnd2(h0, h1);
        float du0 = d0 * sl0, du1 = d1 * sl1;
        duw[i] = rnd2(du0, du1);
        float dg0 = ((d0 * u0) * sg0) * (g0 * (1.0f - sg0) + 1.0f);
        float dg1 = ((d1 * u1) * sg1) * (g1 * (1.0f - sg1) + 1.0f);
        dgw[i] = rnd2(dg0, dg1);
      }
      if (kDgu) {
        uint4* o = reinterpret_cast<uint4*>(dgu_out + (int64_t)mc * 2 * N + jb + lg * 16);
        o[0] = make_uint4(dgw[0], dgw[1], dgw[2], dgw[3]);
        o[1] = make_uint4(dgw[4], dgw[5], dgw[6], dgw[7]);
        uint4* o2 = reinterpret_cast<uint4*>(dgu_out + (int64_t)mc * 2 * N + N + jb + lg * 16);
        o2[0] = make_uint4(duw[0], duw[1], duw[2], duw[3]);
        o2[1] = make_uint4(duw[4], duw[5], duw[6], duw[7]);
      }
      // MX codes of dg and du: stored now, or (kStage) after the row block's barrier
      uint4 cg = {}, cu = {};
      uint32_t eg = 0, eu = 0;
      if (kQuant) {
        eg = quant16_codes(dgw, cg);
        eu = quant16_codes(duw, cu);
        if (!kStage) {
          quant16_store(cg, eg, m, live, q, mc, 2 * N, q_tiled, jb + lg * 16, s, 2 * N / 128);
          quant16_store(cu, eu, m, live, q, mc, 2 * N, q_tiled, N + jb + lg * 16, s, 2 * N / 128);
        }
      }
      if (!live) {  // padded rows add nothing to the sums below
#pragma unroll
        for (int i = 0; i < 8; ++i) dgw[i] = duw[i] = hw[i] = 0u;
      }
      // dxa_g | dxa_u | xS_down products over this tile's columns, D[ρ][m] -> LDS (lane l: m = l % 32,
      // ρ = tile_col(i, l))
      {
        v16f p = v16f{};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fbg[ks], words_bf8(dgw + 4 * ks), p, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int rr = tile_col(i, lane);
          if (rr < R) red[buf][w][lane & 31][rr] = p[i];
        }
        p = v16f{};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fbu[ks], words_bf8(duw + 4 * ks), p, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int rr = tile_col(i, lane);
          if (rr < R) red[buf][w][lane & 31][R + rr] = p[i];
        }
        p = v16f{};
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) p = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fad[ks], words_bf8(hw + 4 * ks), p, 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int rr = tile_col(i, lane);
          if (rr < R) red[buf][w][lane & 31][2 * R + rr] = p[i];
        }
      }
      // dB_g, dB_u, dA_dᵀ: D[j][ρ] += Σ_m dg[m, j] xs_g[m, ρ] etc. over the 32 rows (one k = 32 step)
      // one transpose tile per wave, refilled three times: a wave's LDS operations run in order, so each store
      // follows the reads of the tile's previous contents
      auto tr_pass = [&](const uint32_t* vals, const v8bf* tf, v4f (*acc)[R / 16]) {
        tr_store(trt[w], lane, vals);
#pragma unroll
        for (int jh = 0; jh < 2; ++jh) {
          const v8bf a = tr_operand(trt[w], jh * 16, lane);
#pragma unroll
          for (int h = 0; h < R / 16; ++h) acc[jh][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, tf[h], acc[jh][h], 0, 0, 0);
        }
      };
      if constexpr (kStage) {
#pragma unroll
        for (int h = 0; h < R / 16; ++h) {  // read where used: not held in registers across the block
          tg[h] = sop_read(sb, 3 * (R / 16) + h);
          tu[h] = sop_read(sb, 4 * (R / 16) + h);
          td[h] = sop_read(sb, 5 * (R / 16) + h);
        }
      }
      tr_pass(dgw, tg, dbg);
      tr_pass(duw, tu, dbu);
      tr_pass(hw, td, dad);
      // kStage: this wave's DMA of the next row block's operands has landed (a drain: the count needs no
      // knowledge of what the compiler issued in between; the block's own stores come after the barrier, so
      // only older ones are waited for); after the barrier every wave's DMA has
      if constexpr (kStage) wait_vmcnt<0>();
      // sum the waves' products (fixed order) into the pass's own partial (stores only: a read-modify-write
      // here would wait behind the next row block's prefetch, the memory counter completing in order)
      __syncthreads();
      if (kStage && kQuant) {
        quant16_store(cg, eg, m, live, q, mc, 2 * N, q_tiled, jb + lg * 16, s, 2 * N / 128);
        quant16_store(cu, eu, m, live, q, mc, 2 * N, q_tiled, N + jb + lg * 16, s, 2 * N / 128);
      }
      float* qpart = dxa_part + ((int64_t)(blockIdx.y * (CG / kCols) + oc) * T + rb) * 3 * R;
      for (int idx = threadIdx.x; idx < 32 * 3 * R; idx += 256 * kQ) {
        const int mm = idx / (3 * R), cc = idx % (3 * R);
        float v = red[buf][0][mm][cc];
#pragma unroll
        for (int u = 1; u < kW; ++u) v += red[buf][u][mm][cc];
        if (rb + mm < T) qpart[idx] = v;
      }
      if (kRB == 1) __syncthreads();  // the next row block refills the same buffer
    };
    RowIn b0, b1;  // alternating buffers: no register copies between row blocks
    fetch(r0, b0);
    if constexpr (kStage) {  // the first row block's operands
      stage(r0, 0);
      wait_vmcnt<0>();
      __syncthreads();
    }
    int rb = r0;
    for (; rb + 32 < r1; rb += 64) {
      block(rb, b0, b1, 0);
      block(rb + 32, b1, b0, kRB - 1);
    }
    if (rb < r1) {
      block(rb, b0, b1, 0);
      if (kRB == 2) __syncthreads();  // an odd count: the next pass's first row block refills buffer 0
    }
    if constexpr (kStage) {
      // the last row block's DMA (a repeat of its own operands) has landed in every wave before the next pass
      // stages into either buffer
      wait_vmcnt<0>();
      __syncthreads();
    }
    // dB partials of this super-block: D[j][ρ], lane l: ρ = 16 h + l % 16, j = jb + 16 jh + (l / 16) * 4 + i
#pragma unroll
    for (int jh = 0; jh < 2; ++jh)
#pragma unroll
      for (int h = 0; h < R / 16; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int rr = h * 16 + (lane & 15);
          const int j = jb + jh * 16 + (lane >> 4) * 4 + i;
          dbg_part[((int64_t)blockIdx.x * N + j) * R + rr] = dbg[jh][h][i];
          dbu_part[((int64_t)blockIdx.x * N + j) * R + rr] = dbu[jh][h][i];
          dad_part[((int64_t)blockIdx.x * R + rr) * N + j] = dad[jh][h][i];
        }
  }
}

// out[i] = cast(scale * Σ_p part[p * count + i]), p ascending.  kVec: four outputs per thread with 16-byte loads
// (count % 4 == 0); either way eight partials are loaded before they are added (in order), so a thread waits
// for one memory latency per eight partials, not one per partial.
template <bool kBf16, bool kVec>
__global__ __launch_bounds__(256) void sum_parts_kernel(const float* __restrict__ part, int64_t n_parts,
                                                        int64_t count, float scale, void* __restrict__ out) {
  typedef typename std::conditional<kVec, float4, float>::type F;
  constexpr int kW = kVec ? 4 : 1;
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * kW;
  if (i >= count) return;
  const F* src = reinterpret_cast<const F*>(part + i);
  const int64_t stride = count / kW;  // in units of F
  auto add = [](F& a, const F& b) {
    if constexpr (kVec) {
      a.x += b.x; a.y += b.y; a.z += b.z; a.w += b.w;
    } else {
      a += b;
    }
  };
  F v = src[0];
  int64_t p = 1;
  for (; p + 7 < n_parts; p += 8) {
    F x[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] = src[(p + u) * stride];
#pragma unroll
    for (int u = 0; u < 8; ++u) add(v, x[u]);
  }
  for (; p < n_parts; ++p) add(v, src[p * stride]);
  const float* f = reinterpret_cast<const float*>(&v);
#pragma unroll
  for (int k = 0; k < kW; ++k) {
    const float o = f[k] * scale;
    if (kBf16) reinterpret_cast<uint16_t*>(out)[i + k] = (uint16_t)f32_to_bf16_bits(o);
    else reinterpret_cast<float*>(out)[i + k] = o;
  }
}

}  // namespace

namespace {

int device_cus() {
  int dev = 0, v = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0)
    return 256;
  return v;
}

}  // namespace

extern "C" int64_t mxfp8_mlp_fwd_groups(int64_t T, int64_t N, int64_t r) {
  if (T <= 0 || N <= 0 || N % 128 || (r != 16 && r != 32)) return 0;
  // One wave per (32-row block, column group); a CU holds kFwdWavesPerSimd waves per SIMD.  Every wave of a
  // round runs at the same pace, so the time goes as rounds x (tiles per group + ~1 tile of set-up).  Pick
  // the group count (a divisor of N/32) with the least of that; among ties, the fewest groups (smallest
  // partial-sum buffer).
  const int64_t cap = (int64_t)device_cus() * 4 * kFwdWavesPerSimd, nt = N / 32, nrb = (T + 127) / 128 * 4;
  int64_t best = 1, best_cost = -1;
  for (int64_t g = 1; g <= nt; ++g) {
    if (nt % g) continue;
    const int64_t rounds = (nrb * g + cap - 1) / cap;
    const int64_t cost = rounds * (nt / g + 1);
    if (best_cost < 0 || cost < best_cost) {
      best_cost = cost;
      best = g;
    }
  }
  return best;
}

extern "C" int mxfp8_mlp_fwd(const void* gu, const void* xs, const void* bg, const void* bu, const void* ad, int64_t T,
                             int64_t N, int64_t r, float s_g, float s_u, void* q_h, void* s_h, float* part,
                             int64_t n_groups, void* h_out, int64_t q_layout, void* stream) {
  MX_CHECK_ARG(gu && xs && bg && bu && ad && part, "mxfp8_mlp_fwd: null pointer");
  MX_CHECK_ARG(q_layout >= 0 && q_layout <= 3,
               "mxfp8_mlp_fwd: q_layout must be 0..3 (bit 0: q_h MX-tiled, bit 1: gu in the FT layout)");
  MX_CHECK_ARG((q_h == nullptr) == (s_h == nullptr), "mxfp8_mlp_fwd: q_h and s_h go together");
  MX_CHECK_ARG(!h_out || q_h, "mxfp8_mlp_fwd: h_out needs q_h");
  MX_CHECK_ARG(T > 0 && N > 0 && N % 128 == 0 && (r == 16 || r == 32), "mxfp8_mlp_fwd: bad shape");
  MX_CHECK_ARG(T * 2 * N < (1LL << 31), "mxfp8_mlp_fwd: T * 2N must stay below 2^31");
  MX_CHECK_ARG(n_groups > 0 && (N / 32) % n_groups == 0, "mxfp8_mlp_fwd: n_groups must divide N / 32");
  MX_CHECK_ARG(mx_aligned(gu, 16) && mx_aligned(xs, 16) && mx_aligned(bg, 16) && mx_aligned(bu, 16) &&
                   mx_aligned(ad, 16) && mx_aligned(part, 16) && (!q_h || mx_aligned(q_h, 16)) &&
                   (!h_out || mx_aligned(h_out, 16)),
               "mxfp8_mlp_fwd: misaligned buffer");
  const int64_t Tpad = (T + 127) / 128 * 128;
  dim3 grid((unsigned)(Tpad / 128), (unsigned)n_groups);
  const int tpg = (int)(N / 32 / n_groups);
  hipStream_t stm = (hipStream_t)stream;
#define FWD_ARGS (const uint16_t*)gu, (const uint16_t*)xs, (const uint16_t*)bg, (const uint16_t*)bu, (const uint16_t*)ad, \
                 (int)T, (int)Tpad, (int)N, tpg, s_g, s_u, (uint8_t*)q_h, (uint8_t*)s_h, part, (uint16_t*)h_out, \
                 (q_layout & 1) != 0, (q_layout & 2) != 0
  if (r == 16) {
    if (h_out) fwd_kernel<16, true, true><<<grid, 256, 0, stm>>>(FWD_ARGS);
    else if (q_h) fwd_kernel<16, true, false><<<grid, 256, 0, stm>>>(FWD_ARGS);
    else fwd_kernel<16, false, false><<<grid, 256, 0, stm>>>(FWD_ARGS);
  } else {
    if (h_out) fwd_kernel<32, true, true><<<grid, 256, 0, stm>>>(FWD_ARGS);
    else if (q_h) fwd_kernel<32, true, false><<<grid, 256, 0, stm>>>(FWD_ARGS);
    else fwd_kernel<32, false, false><<<grid, 256, 0, stm>>>(FWD_ARGS);
  }
#undef FWD_ARGS
  MX_CHECK_LAUNCH("mxfp8_mlp_fwd");
  return MXFP8_OK;
}

extern "C" int mxfp8_mlp_bwd(const void* gu, const void* xs, const void* xsT, const void* dhm, const void* dxd,
                             const void* dxdT, const void* bg, const void* bu, const void* bgT, const void* buT,
                             const void* ad, const void* adT, int64_t T, int64_t N, int64_t r, float s_g, float s_u,
                             int64_t SB, int64_t CG, void* q, void* s, float* dxa_part, float* dbg_part,
                             float* dbu_part, float* dad_part, void* dgu_out, int64_t q_layout, void* stream) {
  MX_CHECK_ARG(q_layout >= 0 && q_layout <= 7,
               "mxfp8_mlp_bwd: q_layout must be 0..7 (bit 0: q MX-tiled, bit 1: gu and dhm in the FT layout, bit 2: "
               "8-wave workgroups, one dxa partial per 256 columns)");
  MX_CHECK_ARG(gu && xs && xsT && dhm && dxd && dxdT && bg && bu && bgT && buT && ad && adT && dxa_part &&
                   dbg_part && dbu_part && dad_part,
               "mxfp8_mlp_bwd: null pointer");
  MX_CHECK_ARG((q == nullptr) == (s == nullptr), "mxfp8_mlp_bwd: q and s go together");
  MX_CHECK_ARG(T > 0 && N > 0 && N % 128 == 0 && (r == 16 || r == 32), "mxfp8_mlp_bwd: bad shape (N %% 128)");
  MX_CHECK_ARG(T * 2 * N < (1LL << 31), "mxfp8_mlp_bwd: T * 2N must stay below 2^31");
  const bool wide = (q_layout & 4) != 0;
  MX_CHECK_ARG(SB > 0 && SB % 128 == 0 && CG > 0 && CG % (wide ? 256 : 128) == 0 && N % CG == 0,
               "mxfp8_mlp_bwd: SB must be a multiple of 128, CG a multiple of 128 (256 with bit 2) dividing N");
  MX_CHECK_ARG(!wide || !dgu_out, "mxfp8_mlp_bwd: dgu_out takes the 4-wave workgroups");
  MX_CHECK_ARG(mx_aligned(gu, 16) && mx_aligned(dhm, 16) && mx_aligned(xs, 16) && mx_aligned(xsT, 16) &&
                   mx_aligned(dxd, 16) && mx_aligned(dxdT, 16) && mx_aligned(bg, 16) && mx_aligned(bu, 16) &&
                   mx_aligned(bgT, 16) && mx_aligned(buT, 16) && mx_aligned(ad, 16) && mx_aligned(adT, 16) &&
                   (!q || mx_aligned(q, 16)) && (!dgu_out || mx_aligned(dgu_out, 16)),
               "mxfp8_mlp_bwd: misaligned buffer");
  const int64_t Tpad = (T + 127) / 128 * 128;
  dim3 grid((unsigned)((Tpad + SB - 1) / SB), (unsigned)(N / CG));
  hipStream_t stm = (hipStream_t)stream;
#define BWD_ARGS (const uint16_t*)gu, (const uint16_t*)xs, (const uint16_t*)xsT, (const uint16_t*)dhm, (const uint16_t*)dxd, \
                 (const uint16_t*)dxdT, (const uint16_t*)bg, (const uint16_t*)bu, (const uint16_t*)bgT,                    \
                 (const uint16_t*)buT, (const uint16_t*)ad, (const uint16_t*)adT, (int)T, (int)Tpad, (int)N, (int)SB,     \
                 (int)CG, s_g, s_u, (uint8_t*)q, (uint8_t*)s, dxa_part, dbg_part, dbu_part, dad_part, (uint16_t*)dgu_out, \
                 (q_layout & 1) != 0, (q_layout & 2) != 0
  MX_CHECK_ARG(!dgu_out || q, "mxfp8_mlp_bwd: dgu_out needs q");
  if (wide) {
    if (r == 16) {
      if (q) bwd_kernel<16, true, false, 2><<<grid, 512, 0, stm>>>(BWD_ARGS);
      else bwd_kernel<16, false, false, 2><<<grid, 512, 0, stm>>>(BWD_ARGS);
    } else {
      if (q) bwd_kernel<32, true, false, 2><<<grid, 512, 0, stm>>>(BWD_ARGS);
      else bwd_kernel<32, false, false, 2><<<grid, 512, 0, stm>>>(BWD_ARGS);
    }
  } else if (r == 16) {
    if (dgu_out) bwd_kernel<16, true, true><<<grid, 256, 0, stm>>>(BWD_ARGS);
    else if (q) bwd_kernel<16, true, false><<<grid, 256, 0, stm>>>(BWD_ARGS);
    else bwd_kernel<16, false, false><<<grid, 256, 0, stm>>>(BWD_ARGS);
  } else {
    if (dgu_out) bwd_kernel<32, true, true><<<grid, 256, 0, stm>>>(BWD_ARGS);
    else if (q) bwd_kernel<32, true, false><<<grid, 256, 0, stm>>>(BWD_ARGS);
    else bwd_kernel<32, false, false><<<grid, 256, 0, stm>>>(BWD_ARGS);
  }
#undef BWD_ARGS
  MX_CHECK_LAUNCH("mxfp8_mlp_bwd");
  return MXFP8_OK;
}

extern "C" int mxfp8_sum_parts(const float* part, int64_t n_parts, int64_t count, float scale, void* out,
                               int out_bf16, void* stream) {
  MX_CHECK_ARG(part && out && n_parts > 0 && count >= 0, "mxfp8_sum_parts: bad arguments");
  if (count == 0) return MXFP8_OK;
  const bool vec = count % 4 == 0 && mx_aligned(part, 16);
  const int64_t blocks = (count / (vec ? 4 : 1) + 255) / 256;
  MX_CHECK_ARG(blocks < (1LL << 31), "mxfp8_sum_parts: too large");
  hipStream_t stm = (hipStream_t)stream;
  if (vec) {
    if (out_bf16) sum_parts_kernel<true, true><<<(unsigned)blocks, 256, 0, stm>>>(part, n_parts, count, scale, out);
    else sum_parts_kernel<false, true><<<(unsigned)blocks, 256, 0, stm>>>(part, n_parts, count, scale, out);
  } else {
    if (out_bf16) sum_parts_kernel<true, false><<<(unsigned)blocks, 256, 0, stm>>>(part, n_parts, count, scale, out);
    else sum_parts_kernel<false, false><<<(unsigned)blocks, 256, 0, stm>>>(part, n_parts, count, scale, out);
  }
  MX_CHECK_LAUNCH("mxfp8_sum_parts");
  return MXFP8_OK;
}
