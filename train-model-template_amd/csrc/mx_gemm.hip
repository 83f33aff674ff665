// MX block-scaled GEMM for gfx950: C[M, N] = bf16(A[M, K] · B[N, K]ᵀ), E4M3 operands with E8M0 scales per 32
// elements along K, fp32 accumulation on v_mfma_scale_f32_32x32x64_f8f6f4, optional rank-r bf16 epilogue.
//
// Replaces torch._scaled_mm (cuBLAS block-scaled GEMM) at /root/reference/scripts/fused_mlp.py:279, :283, :309,
// :329 and the addmm_ epilogues at :284 and :331.
//
// Tiling: a workgroup computes a 256 (M) x 128 (N) tile with four waves, two workgroups per CU (kNW = 1;
// layout bit MXFP8_GEMM_WIDE selects the 8-wave 256 x 256 shape, kNW = 2, one workgroup per CU), in K steps
// of 64 (two scale blocks).  Measured on the four MLP GEMMs (T=10752, d=2048, f=6144): 845-858 us at
// kNW = 1 against 873-908 us at kNW = 2 with its best tail split.  Each wave
// holds a 64 (M) x 128 (N) sub-tile as a 2 x 4 grid of 32 x 32 MFMA tiles (128 accumulators per lane), so two
// waves share each SIMD; with two independent workgroups per CU one workgroup's pipeline fill, barrier waits
// and epilogue overlap the other's matrix work.  The matrix instruction takes the weight (B) fragment as its
// first operand, so each lane's accumulators cover one output row m and 16 columns n in runs of 4.
//
// What bounds it (rocprofv3 counters on the MLP GEMMs): the CU's vector-memory path that carries the
// operand DMA (TA / TD busy 65-89% of the kernel, TD waiting on L1/L2 data about 45% of the time) while the
// matrix pipe is busy ~48%.  LDS reads overlap MFMAs well on gfx950 (a software-pipelined fragment-read +
// MFMA loop runs at 94-97% of the MFMA-only rate), and an L2 prefetch ahead of the ring made it slower.
//
// Operand layouts: row-major codes (row stride lda / ldb), or the MX-tiled layout (tiled_offset in
// mx_device.h) in which each 16-row x 64-code slice is one contiguous 1 KB block in LDS order.  The GEMM is
// bound by how fast the DMA brings operands from L2: measured with the MFMAs removed, the tiled layout moves
// the same bytes in ~0.7x the time of the row-major one (64-byte row pieces use half of each 128-byte line
// per request), and the full GEMM gains 10-25%.  Both layouts leave the same bytes in LDS, so results are
// bit-identical.
//
// Operand staging: global memory goes straight into LDS with global_load_lds_dwordx4 (no VGPR round trip)
// through a ring of 3 stages of 26 KB (kNW = 2: 4 of 34 KB): A codes 256 x 64 B, B codes 128 x 64 B, and the
// 128-row blocked scale tiles of each operand for the current 128-wide K tile.  Every wave issues the same
// number of DMA instructions per stage (1 KB code slices of A and of B plus a scale tile or a duplicate), so a
// fixed vmcnt bounds the wait for a stage while the later ones stay in flight.  Lane i of a DMA lands at
// base + 16 i; a row's 16-byte chunk c is stored at chunk c ^ ((row >> 2) & 3): the gfx950 LDS serves a
// ds_read_b128 16 lanes (16 consecutive rows, same chunk) at a time over 64 banks, and with 64-byte rows
// rows r, r+4, r+8, r+12 share bank groups unless their chunks differ (measured: 48% bank-conflict cycles
// with a (row >> 1) swizzle).
// Scale words: for a 32-row group the 16 bytes at (row % 32) * 16 of a blocked tile hold the four 32-row
// groups' scales for one 128-wide K tile; a lane shifts its word by 8 * (lane / 32) so that op_sel 0 / 2
// selects block 2P + lane/32 of the current half-tile P.
// Work order: a 1-D grid in which workgroup i runs on XCD i % 8 (the dispatcher's round robin).  Tiles are
// numbered in groups of kGroupM M-tiles (M fastest inside a group) and each XCD takes a contiguous range of
// that order, so the tiles resident on one XCD share A and B panels in its L2.  With the 8-wave shape, when
// the last wave of tiles would fill at most half of the CUs, those tail tiles are split along K into `parts`
// pieces run as separate workgroups after the full tiles; each piece writes its fp32 accumulators to the
// caller's workspace, and the piece that arrives last (agent-scope counter) adds the pieces in part order,
// which makes the result independent of arrival order, runs the epilogue and resets its counter to zero.
#include <algorithm>
#include <atomic>
#include <mutex>
#include <type_traits>

#include "abi_common.h"
#include "mx_device.h"
#include "presum_device.h"
#include "tn_device.h"

// gu leaves the gate|up epilogue with non-temporal stores: it is read again only by the backward, and
// streaming it past the last-level cache keeps MX(h) and the xS_down partials there for the down GEMM and the
// partial sum that follow (with the backward's non-temporal gu loads, MX_BWD_NT_LOAD in mlp_fused.hip: 10-17 us
// per configuration-3 step faster over five A/B pairs on one box).
#ifndef MX_NT_GU
#define MX_NT_GU 1
#endif

using namespace mxk;

namespace {

constexpr int kBM = 256, kBK = 64;
constexpr int kCodeBytes = kBM * kBK;  // A codes per stage: 16 KB
constexpr int kGroupM = 4;
constexpr int kMaxParts = 4;
// Workspace layout: arrival counters at a fixed place (so every shape finds its own counters at zero, each
// launch resets those it used), fp32 partial tiles after them.
constexpr int64_t kCounterBytes = 4096;
constexpr int kMaxSplitTiles = (int)(kCounterBytes / 4);

// Workgroup shapes.  kNW = 2: 8 waves, 256 x 256 tile, 4-stage ring of 34 KB (one workgroup per CU).
// kNW = 1: 4 waves, 256 x 128 tile, 3-stage ring of 26 KB (two workgroups per CU, whose barriers are
// independent, so one workgroup's MFMAs fill the other's waits).  Every wave computes a 64 (M) x 128 (N)
// sub-tile either way.
template <int kNW>
struct Shape {
  static constexpr int kWaves = 4 * kNW, kThreads = 64 * kWaves, kBN = 128 * kNW;
  static constexpr int kStages = kNW == 2 ? 4 : 3;
  static constexpr int kOffA = 0, kOffB = kCodeBytes, kOffSA = kCodeBytes + kBN * kBK, kOffSB = kOffSA + 1024;
  static constexpr int kStageBytes = kOffSB + 1024;
  // DMA per wave and stage: kSA 1 KB slices of A, kSB of B, and one more (A's or B's scale tiles, or a
  // repeat of the wave's last B slice), so a fixed vmcnt bounds every wait.
  static constexpr int kSA = 16 / kWaves, kSB = (kBN / 16) / kWaves, kDma = kSA + kSB + 1;
  static constexpr int64_t kPartBytes = (int64_t)kBM * kBN * 4;  // fp32 partial tile
};

struct Lora {
  const uint16_t* p;  // [M, r] bf16
  int64_t ld_p;
  const uint16_t* q;  // [N, r] bf16
  int64_t ld_q;
  float alpha;
};

// Fused SwiGLU forward epilogue (kEpi == kEpiSwiGluFwd): the operands beyond the GEMM's.  The B operand is
// W_gu = [W_gate; W_up] in the fused row order (fused_swiglu_row in the host code): output tile t (128 columns) holds gate columns
// 64 t + 0..63 and then up columns 64 t + 0..63, each 32-column block with its weight rows permuted by pi_col,
// so that acc[b][mt] (gate) and acc[2 + b][mt] (up) hold, in lane l, row m = l % 32 and the 16 CONTIGUOUS
// columns jb + (l / 32) * 16 + i (jb = 64 t + 32 b): the layout of the fused forward kernel and of the FT blocks.
struct SwEpi {
  const uint16_t* xs;  // [M, 2r] bf16: x · [A_g; A_u]ᵀ
  const uint16_t* bg;  // [N, r] bf16 LoRA B of gate
  const uint16_t* bu;  // [N, r] bf16 LoRA B of up
  const uint16_t* ad;  // [r, N] bf16 LoRA A of down
  float s_g, s_u;
  uint16_t* gu;        // [ceil(M/32)*32, 2N] bf16 GEMM output (gate | up), fused-tile layout
  uint8_t* q;          // [ceil(M/16)*16, N] MX-tiled codes of h
  uint8_t* s;          // blocked scales of h (ceil(M/128) tile rows, N/128 tiles)
  float* part;         // [2N/128, M, r] xS_down partials, one per output tile
  int N;               // d_ffn
};

// Fused SwiGLU backward epilogue (kEpi == kEpiSwiGluBwd).  The GEMM is dhm = MX(dy) · W_down with B = W_downᵀ
// [N, K] in the dgrad row order (fused_dgrad_row in the host code: inside each 32-row block row a is logical row
// pi_col(a)), so that acc[nt][mt] holds, in lane l, row m = l % 32 and the 16 contiguous columns
// n0 + 32 nt + (l / 32) * 16 + i, the lane layout of the fused backward kernel.  The epilogue is that kernel's
// per-tile work (mlp_fused.hip, bwd_kernel) with dhm taken from the accumulators instead of memory.
struct SwBwd {
  const uint16_t* gu;    // [ceil(M/32)*32, 2N] bf16 saved gate | up GEMM output, fused-tile layout
  const uint16_t* xs;    // [M, 2r] bf16: x · [A_g; A_u]ᵀ
  const uint16_t* xsT;   // [2r, Tpad] its transpose, zero past M (Tpad = ceil(M/128)*128)
  const uint16_t* dxd;   // [M, r] bf16(bf16(dy · B_d) s_d)
  const uint16_t* dxdT;  // [r, Tpad] its transpose, zero past M
  const uint16_t* bg;    // [N, r] LoRA B of gate, and its transpose bgT [r, N]
  const uint16_t* bgT;
  const uint16_t* bu;    // [N, r] LoRA B of up, and buT [r, N]
  const uint16_t* buT;
  const uint16_t* ad;    // [r, N] LoRA A of down, and adT [N, r]
  const uint16_t* adT;
  float s_g, s_u;
  uint8_t* q;            // [ceil(M/16)*16, 2N] MX-tiled codes of dg | du (the dgrad GEMM's A operand)
  uint8_t* s;            // their blocked scales (ceil(M/128) tile rows, 2N/128 tiles)
  float* dxa;            // [N/128, M, 3r] partials dxa_g | dxa_u | xS_down, one per output tile
  float* dbg;            // [ceil(M/256), N, r] dB_g partials, one per tile row
  float* dbu;            // [ceil(M/256), N, r] dB_u partials
  float* dad;            // [ceil(M/256), r, N] dA_d partials
};

constexpr int kEpiPlain = 0, kEpiSwiGluFwd = 1, kEpiSwiGluBwd = 2;
// LDS of the backward epilogue (r = 16), in the operand ring:
//   per wave three [32][kTrLd] bf16 transpose tiles (dg, du, h), which afterwards carry the wave's dB_g, dB_u,
//   dA_dᵀ sums of the block (3 x [32 x 16] fp32) to the cross-wave reduction;
//   the tile's dB_g, dB_u, dA_d sums over its first row blocks, [4 column blocks][3][512] fp32;
//   the tile's LoRA weights, bf16: rows n0..n0+127 of B_g, B_u, A_dᵀ ([128][16] each) and the same columns of
//   B_gᵀ, B_uᵀ, A_d ([16][128] each).
constexpr int kBwdTrBytes = 3 * 32 * kTrLd * 2;
constexpr int kBwdDbOff = 4 * kBwdTrBytes, kBwdDbBytes = 4 * 3 * 512 * 4;
constexpr int kBwdWOff = kBwdDbOff + kBwdDbBytes, kBwdWBytes = 6 * 128 * 16 * 2;
static_assert(kBwdWOff + kBwdWBytes <= Shape<1>::kStages * Shape<1>::kStageBytes, "backward epilogue LDS");
static_assert(3 * 32 * 16 * 4 <= kBwdTrBytes, "dB exchange fits a wave's transpose tiles");

// Output columns in up to four segments, each its own row-major matrix: columns [col0[k], col0[k + 1]) of the
// product go to ptr[k] with row stride ld[k] (segment boundaries are multiples of the tile width, so a tile
// writes into one segment).  One segment = the plain C, ldc.
struct CSeg {
  int n;
  int col0[4];
  int64_t ld[4];
  uint16_t* ptr[4];
  int rcol[4];  // first column of P and Q of the segment's rank-r product (0 unless mxfp8_gemm_nt_seg sets it)
};

// Launch plan (computed on the host, see make_plan).
struct Plan {
  int tm, tn;        // tiles along M and N
  int full;          // logical tiles [0, full) run whole
  int per_full;      // full tiles per XCD (ceil(full / 8)); grid part one = 8 * per_full workgroups
  int nsplit;        // logical tiles [full, full + nsplit) split along K
  int parts;         // pieces per split tile
  int chunk;         // K steps per piece (even)
  int per_split;     // pieces per XCD (ceil(nsplit * parts / 8))
  float4* ws;        // [nsplit][parts][8 waves][32][64 lanes] float4 partial accumulators
  int* cnt;          // [nsplit] arrival counters (zero between launches)
};

__device__ __forceinline__ void tile_coords(int t, int tm, int tn, int& mt, int& nt) {
  const int g = t / (kGroupM * tn), r = t - g * (kGroupM * tn);
  const int rows = min(kGroupM, tm - g * kGroupM);
  mt = g * kGroupM + r % rows;
  nt = r / rows;
}

// The instances that can run token reductions past their tiles (mxfp8_gemm_nt_tn): the plain 4-wave GEMM with
// the rank-16, 32 or 48 LoRA epilogue, the dx GEMMs of the fused MLP (r = 32 at r = 16 adapters) and of the
// grouped linears (q|k|v: 48, o_proj: 16).  At configuration 3 each has 672 tiles, 1.3 rounds of the workgroup
// slots.  Other instances do not compile the reduction.
template <int kR, int kNW, int kEpi>
constexpr bool kFoldTn = (kR == 16 || kR == 32 || kR == 48) && kNW == 1 && kEpi == 0;
// The instance whose epilogue operand P can be summed in its own launch (mxfp8_gemm_nt_sum): the plain 4-wave GEMM
// with the rank-16 epilogue, the fused MLP's down GEMM at r = 16.
template <int kR, int kNW, int kEpi>
constexpr bool kFoldSum = kR == 16 && kNW == 1 && kEpi == 0;
static_assert(tn_batch_lds_elems<true>() * 2 <= 3 * 26 * 1024,
              "the folded token reduction borrows the 4-wave ring's LDS");

// 32 bytes of one operand row for the stage's 64-wide K step: chunk c0 (k 16*(l/32)..) and c0 + 2 (k 32 + ..)
__device__ __forceinline__ v8i frag(const uint8_t* base, int row, int c0, int sw) {
  uint4 lo = *reinterpret_cast<const uint4*>(base + row * kBK + ((c0 ^ sw) << 4));
  uint4 hi = *reinterpret_cast<const uint4*>(base + row * kBK + (((c0 + 2) ^ sw) << 4));
  v8i r;
  r[0] = lo.x; r[1] = lo.y; r[2] = lo.z; r[3] = lo.w;
  r[4] = hi.x; r[5] = hi.y; r[6] = hi.z; r[7] = hi.w;
  return r;
}

template <int kR, int kNW, int kEpi>
__global__ __launch_bounds__(Shape<kNW>::kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void gemm_kernel(
    const uint8_t* __restrict__ A, const uint8_t* __restrict__ SA, int64_t lda, const uint8_t* __restrict__ B,
    const uint8_t* __restrict__ SB, int64_t ldb, int M, int N, int K, CSeg cseg, Lora lora, Plan plan, int tiled,
    SwEpi swe, SwBwd swb, const TnBatch tnb, const PreSum pre) {
  using S = Shape<kNW>;
  __shared__ __attribute__((aligned(16))) uint8_t lds[S::kStages * S::kStageBytes];
  __shared__ int arrived;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (SGPR)
  const int wn = wave >> 2, wm = wave & 3;  // compute sub-tile: n rows wn*128 + [0,128), m rows wm*64 + [0,64)

  // ---- workgroups before the tiles: the sum of the epilogue operand P (mxfp8_gemm_nt_sum, presum_device.h)
  int bid = blockIdx.x;
  if constexpr (kFoldSum<kR, kNW, kEpi>) {
    if (bid < pre.blocks) {
      presum_block(pre, bid);
      return;
    }
    bid -= pre.blocks;  // a multiple of 8: the tiles keep their XCDs
  }

  // ---- workgroups past the tiles: the folded token reductions (mxfp8_gemm_nt_tn), in the ring's LDS.  They are
  // numbered after every tile, so the dispatcher starts them only once each tile has started, in the slots the
  // last round of tiles leaves free.
  if constexpr (kFoldTn<kR, kNW, kEpi>) {
    const int first = 8 * (plan.per_full + plan.per_split);
    if (bid >= first) {
      uint16_t* tl = reinterpret_cast<uint16_t*>(lds);
      if (tnb.kd == 2) tn_batch_block<2, true>(tnb, bid - first, tl);
      else tn_batch_block<1, true>(tnb, bid - first, tl);
      return;
    }
  }

  // ---- which tile (and which K piece) this workgroup computes
  const int ns_all = K / kBK;  // even: K % 128 == 0
  int tile, part = -1, s_begin = 0, s_end = ns_all;
  {
    const int i = bid, x = i & 7, j = i >> 3;
    if (i < 8 * plan.per_full) {
      tile = x * plan.per_full + j;
      if (tile >= plan.full) return;
    } else {
      const int jj = (i - 8 * plan.per_full) >> 3;
      const int u = x * plan.per_split + jj;
      if (jj >= plan.per_split || u >= plan.nsplit * plan.parts) return;
      tile = plan.full + u / plan.parts;
      part = u % plan.parts;
      s_begin = part * plan.chunk;
      s_end = min(ns_all, s_begin + plan.chunk);
    }
  }
  int mt_, nt_;
  tile_coords(tile, plan.tm, plan.tn, mt_, nt_);
  const int m0 = mt_ * kBM, n0 = nt_ * S::kBN;
  const int nkt = K / 128;

  // DMA roles: wave w stages A rows w*16*kSA + [0, 16*kSA) and B rows w*16*kSB + [0, 16*kSB) in 1 KB slices
  // (16 rows x 64 B).  Row-major operand: lane -> row slice*16 + lane/4, logical chunk chosen so that the
  // lane's 16 bytes land at their swizzled LDS position.  MX-tiled operand (tiled_offset in mx_device.h): the
  // slice is one contiguous 1 KB block already in LDS order, lane i copies bytes 16i..16i+15, and a K step
  // advances 1 KB instead of 64 B.
  const bool a_tiled = tiled & 1, b_tiled = (tiled >> 1) & 1, c_ft = (tiled >> 3) & 1, b_pi = (tiled >> 4) & 1;
  const int kst = K / kBK;
  const int lchunk = (lane & 3) ^ ((lane >> 4) & 3);  // (row >> 2) & 3 == (lane >> 4) & 3 for these rows
  auto slice_off = [&](bool op_tiled, int R0, int Rn, int64_t ldd, int rbase) -> uint32_t {
    if (op_tiled) {
      const int rg = min((R0 >> 4) + (rbase >> 4), ((Rn + 15) >> 4) - 1) - (R0 >> 4);  // clamp past the end
      return (uint32_t)(rg * kst * 1024) + lane * 16;
    }
    const int row = rbase + (lane >> 2);
    return (uint32_t)((min(R0 + row, Rn - 1) - R0) * ldd) + lchunk * 16;  // clamp rows past the end
  };
  const uint8_t* ga = A + (a_tiled ? (int64_t)(m0 >> 4) * kst * 1024 : (int64_t)m0 * lda);
  const uint8_t* gb = B + (b_tiled ? (int64_t)(n0 >> 4) * kst * 1024 : (int64_t)n0 * ldb);
  const int sa_stride = a_tiled ? 1024 : kBK, sb_stride = b_tiled ? 1024 : kBK;
  uint32_t goa[S::kSA], gob[S::kSB];
#pragma unroll
  for (int j = 0; j < S::kSA; ++j) goa[j] = slice_off(a_tiled, m0, M, lda, (wave * S::kSA + j) * 16);
#pragma unroll
  for (int j = 0; j < S::kSB; ++j) gob[j] = slice_off(b_tiled, n0, N, ldb, (wave * S::kSB + j) * 16);
  // Last DMA of the stage, without divergence: wave 0 copies A's two 128-row scale tiles, wave 1 B's
  // scale tile(s) (1 KB, lane -> tile lane / 32, bytes (lane % 32) * 16 of it; for a 128-row B tile the
  // upper half holds the next tile's, unused); the other waves repeat their last B slice (same source, same
  // destination: a harmless duplicate).
  const bool scl = wave < 2;
  const int sR0 = wave == 0 ? m0 : n0, sRn = wave == 0 ? M : N;
  const int stile = min((sR0 >> 7) + (lane >> 5), (sRn - 1) >> 7);
  const uint8_t* sgp = (wave == 0 ? SA : SB) + (int64_t)stile * nkt * 512 + (lane & 31) * 16;
  const int dma_a_off = S::kOffA + wave * S::kSA * 1024, dma_b_off = S::kOffB + wave * S::kSB * 1024;
  const int dma_x_off = wave == 0 ? S::kOffSA : wave == 1 ? S::kOffSB : dma_b_off + (S::kSB - 1) * 1024;

  const uint32_t lds0 = lds_addr(lds);
  const int last = s_end - 1;
  auto issue_to = [&](int s, int slot) {  // DMA stage s into ring slot `slot`
    const uint32_t st = lds0 + slot * S::kStageBytes;
    const uint8_t* pa = ga + s * sa_stride;
    const uint8_t* pb = gb + s * sb_stride;
#pragma unroll
    for (int j = 0; j < S::kSA; ++j) dma16(pa + goa[j], st + dma_a_off + j * 1024);
#pragma unroll
    for (int j = 0; j < S::kSB; ++j) dma16(pb + gob[j], st + dma_b_off + j * 1024);
    dma16(scl ? sgp + (s >> 1) * 512 : pb + gob[S::kSB - 1], st + dma_x_off);
  };

  v16f acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc[i][0] = v16f{};
    acc[i][1] = v16f{};
  }

  const int sshift = (lane >> 5) * 8;
  const int sw = (lane >> 2) & 3;  // swizzle of rows base + lane % 32 (base a multiple of 32)
  const int c0 = lane >> 5;
  struct Frags {
    v8i a0, a1, b0, b1, b2, b3;
    uint2 sa;
    uint4 sb;
  };
  auto read = [&](int slot, Frags& f) {
    const uint8_t* st = lds + slot * S::kStageBytes;
    f.sa = *reinterpret_cast<const uint2*>(st + S::kOffSA + (wm >> 1) * 512 + (lane & 31) * 16 + (wm & 1) * 8);
    f.sb = *reinterpret_cast<const uint4*>(st + S::kOffSB + wn * 512 + (lane & 31) * 16);
    const uint8_t* la = st + S::kOffA;
    const uint8_t* lb = st + S::kOffB;
    f.a0 = frag(la, wm * 64 + (lane & 31), c0, sw);
    f.a1 = frag(la, wm * 64 + 32 + (lane & 31), c0, sw);
    f.b0 = frag(lb, wn * 128 + (lane & 31), c0, sw);
    f.b1 = frag(lb, wn * 128 + 32 + (lane & 31), c0, sw);
    f.b2 = frag(lb, wn * 128 + 64 + (lane & 31), c0, sw);
    f.b3 = frag(lb, wn * 128 + 96 + (lane & 31), c0, sw);
  };
  auto mma = [&](const Frags& f, auto pc) {
    constexpr int P = decltype(pc)::value;  // half of the 128-wide K tile: blocks 2P, 2P + 1
    const int sa0 = (int)(f.sa.x >> sshift), sa1 = (int)(f.sa.y >> sshift);
    const int sb0 = (int)(f.sb.x >> sshift), sb1 = (int)(f.sb.y >> sshift);
    const int sb2 = (int)(f.sb.z >> sshift), sb3 = (int)(f.sb.w >> sshift);
    acc[0][0] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.b0, f.a0, acc[0][0], 0, 0, 2 * P, sb0, 2 * P, sa0);
    acc[0][1] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.b0, f.a1, acc[0][1], 0, 0, 2 * P, sb0, 2 * P, sa1);
    acc[1][0] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.b1, f.a0, acc[1][0], 0, 0, 2 * P, sb1, 2 * P, sa0);
    acc[1][1] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.b1, f.a1, acc[1][1], 0, 0, 2 * P, sb1, 2 * P, sa1);
    acc[2][0] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.b2, f.a0, acc[2][0], 0, 0, 2 * P, sb2, 2 * P, sa0);
    acc[2][1] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.b2, f.a1, acc[2][1], 0, 0, 2 * P, sb2, 2 * P, sa1);
    acc[3][0] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.b3, f.a0, acc[3][0], 0, 0, 2 * P, sb3, 2 * P, sa0);
    acc[3][1] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f.b3, f.a1, acc[3][1], 0, 0, 2 * P, sb3, 2 * P, sa1);
  };
  // Steady state, branch-free (with conditional blocks the compiler sinks a stage's MFMAs below the next
  // barrier).  Step s: wait until stage s + 1 has landed (this wave's DMA) and this wave's reads of stage s are
  // in registers, barrier, refill the slot of stage s with stage s + kStages, read stage s + 1's fragments,
  // then run stage s's MFMAs from registers, so LDS latency and the DMA issue overlap the matrix work.  Every
  // step issues kDma DMA instructions per wave; stages past the end re-load the last stage into the slot just
  // consumed (no later step reads it), so exactly kStages - 2 stages are in flight behind the one waited for.
  int slot = 0;  // ring slot of stage s (wave-uniform)
  auto step = [&](int s, Frags& cur, Frags& nxt, auto pc) {
    wait_vmcnt<(S::kStages - 2) * S::kDma>();
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    // Bare s_barrier: __syncthreads() adds a workgroup fence that waits for every outstanding DMA
    // (vmcnt(0)), which would drain the ring.
    __builtin_amdgcn_s_barrier();
    issue_to(min(s + S::kStages, last), slot);
    slot = slot + 1 == S::kStages ? 0 : slot + 1;
    read(slot, nxt);
    mma(cur, pc);
    __builtin_amdgcn_sched_barrier(0);
  };

#pragma unroll
  for (int q = 0; q < S::kStages; ++q) issue_to(min(s_begin + q, last), q);
  wait_vmcnt<(S::kStages - 1) * S::kDma>();  // stage s_begin landed
  __builtin_amdgcn_s_barrier();
  Frags f0, f1;
  read(0, f0);
  for (int s = s_begin; s < s_end; s += 2) {
    step(s, f0, f1, std::integral_constant<int, 0>{});
    step(s + 1, f1, f0, std::integral_constant<int, 1>{});
  }
  wait_vmcnt<0>();  // drain the redundant tail loads before the workgroup can exit

  if (part >= 0) {
    // split tile: publish this piece, and let the last piece to arrive finish the tile
    const int st_ = tile - plan.full;
    float4* wsp = plan.ws + (((int64_t)st_ * plan.parts + part) * S::kWaves + wave) * (32 * 64) + lane;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          wsp[((i * 2 + j) * 4 + q) * 64] =
              make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]);
    __syncthreads();  // every wave's stores have completed (workgroup release)
    if (tid == 0)
      arrived = __hip_atomic_fetch_add(plan.cnt + st_, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (arrived != plan.parts - 1) return;
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");  // see the other pieces' stores
    const float4* wsb = plan.ws + ((int64_t)st_ * plan.parts * S::kWaves + wave) * (32 * 64) + lane;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
          for (int p = 0; p < plan.parts; ++p) {
            const float4 v = p == part ? make_float4(acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2],
                                                     acc[i][j][4 * q + 3])
                                       : wsb[(int64_t)p * S::kWaves * 32 * 64 + ((i * 2 + j) * 4 + q) * 64];
            if (p == 0) {
              t = v;
            } else {
              t.x += v.x; t.y += v.y; t.z += v.z; t.w += v.w;
            }
          }
          acc[i][j][4 * q] = t.x; acc[i][j][4 * q + 1] = t.y; acc[i][j][4 * q + 2] = t.z;
          acc[i][j][4 * q + 3] = t.w;
        }
    if (tid == 0) __hip_atomic_store(plan.cnt + st_, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  if constexpr (kEpi == kEpiSwiGluFwd) {
    // SwiGLU forward (fused_mlp.py:65-109, the _fwd_kernel math): gu = bf16(acc) is stored as the saved GEMM
    // output, then g = bf16(gu_g + s_g xs_g·B_gᵀ), u = bf16(gu_u + s_u xs_u·B_uᵀ), h = bf16(silu(g) u), MX(h)
    // into the down GEMM's operand and the tile's xS_down partial h·A_dᵀ, per 32 x 32 block of the wave.
    // Every small operand of the tile is loaded first, at once (the main loop's fragment registers are free
    // now), so the epilogue waits for one memory latency instead of one per product.
    constexpr int R = kR, H = R / 16;
    const int Nf = swe.N, lg = lane >> 5, rho = lane & 31;
    const int t64 = n0 >> 1;                      // first gate / up column of the tile: 64 * (n0 / 128)
    const int srows = (M + 127) / 128 * 128;      // rows of the blocked scale buffer of h
    v8bf xg[2][H], xu[2][H], wg[2][H], wu[2][H], af[2][2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int mc = min(m0 + wm * 64 + mt * 32 + (lane & 31), M - 1);
#pragma unroll
      for (int h = 0; h < H; ++h) {
        xg[mt][h] = load_bf8(swe.xs + (int64_t)mc * 2 * R + h * 16 + lg * 8);
        xu[mt][h] = load_bf8(swe.xs + (int64_t)mc * 2 * R + R + h * 16 + lg * 8);
      }
    }
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int jb = t64 + 32 * b;
      const int64_t wr = (int64_t)(jb + pi_col(lane & 31)) * R + lg * 8;
#pragma unroll
      for (int h = 0; h < H; ++h) {
        wg[b][h] = load_bf8(swe.bg + wr + h * 16);
        wu[b][h] = load_bf8(swe.bu + wr + h * 16);
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {  // A_d[ρ, jb + lg*16 + 8 ks + 0..7], ρ = lane % 32 (zero rows past r)
        const v8bf a = load_bf8(swe.ad + (int64_t)(rho < R ? rho : 0) * Nf + jb + lg * 16 + 8 * ks);
        af[b][ks] = rho < R ? a : v8bf{};
      }
    }
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int m = m0 + wm * 64 + mt * 32 + (lane & 31);
      const bool live = m < M;
      v16f xacc = v16f{};  // xS_down partial D[ρ][m] over the tile's 64 columns
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        const int jb = t64 + 32 * b;
        uint32_t gw[8], hw[8];  // gate, then g; up, then u, then h (packed bf16 pairs, columns lg*16 + 2k, +1)
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          float g0 = acc[b][mt][2 * k], g1 = acc[b][mt][2 * k + 1];
          float u0 = acc[2 + b][mt][2 * k], u1 = acc[2 + b][mt][2 * k + 1];
          gw[k] = rnd2(g0, g1);
          hw[k] = rnd2(u0, u1);
        }
        if (live) {  // the lane's columns i = 0..7 and 8..15 are 16 contiguous bytes each in an FT block
          uint16_t* pg = swe.gu + ft_offset(m, jb + lg * 16, 2 * Nf);
          uint16_t* pu = swe.gu + ft_offset(m, Nf + jb + lg * 16, 2 * Nf);
          store_codes<MX_NT_GU>(reinterpret_cast<uint8_t*>(pg), make_uint4(gw[0], gw[1], gw[2], gw[3]));
          store_codes<MX_NT_GU>(reinterpret_cast<uint8_t*>(pg + 512), make_uint4(gw[4], gw[5], gw[6], gw[7]));
          store_codes<MX_NT_GU>(reinterpret_cast<uint8_t*>(pu), make_uint4(hw[0], hw[1], hw[2], hw[3]));
          store_codes<MX_NT_GU>(reinterpret_cast<uint8_t*>(pu + 512), make_uint4(hw[4], hw[5], hw[6], hw[7]));
        }
        {
          const v16f d = lora_pi<R>(wg[b], xg[mt]);
#pragma unroll
          for (int i = 0; i < 16; i += 2) {
            float g0 = bf16_lo(gw[i / 2]) + swe.s_g * d[i], g1 = bf16_hi(gw[i / 2]) + swe.s_g * d[i + 1];
            gw[i / 2] = rnd2(g0, g1);
          }
        }
        {
          const v16f d = lora_pi<R>(wu[b], xu[mt]);
#pragma unroll
          for (int i = 0; i < 16; i += 2) {
            float u0 = bf16_lo(hw[i / 2]) + swe.s_u * d[i], u1 = bf16_hi(hw[i / 2]) + swe.s_u * d[i + 1];
            hw[i / 2] = rnd2(u0, u1);
          }
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const float g0 = bf16_lo(gw[k]), g1 = bf16_hi(gw[k]);
          float h0 = (g0 * fast_sigmoid(g0)) * bf16_lo(hw[k]), h1 = (g1 * fast_sigmoid(g1)) * bf16_hi(hw[k]);
          hw[k] = rnd2(h0, h1);
        }
        {  // MX(h): the lane's 16 codes (one 16-byte piece of the MX-tiled operand) and the block's scale byte
          uint4 c;
          const uint32_t e = quant16_codes(hw, c);
          if (live) store_codes<MX_NT_FUSED>(swe.q + tiled_offset(m, jb + lg * 16, Nf), c);
          if (lg == 0 && m < srows)
            store_scale<MX_NT_FUSED>(swe.s + blocked_offset(m, jb >> 5, Nf / 128), live ? (uint8_t)e : (uint8_t)0);
        }
        // xS_down: D[ρ][m] += Σ_j A_d[ρ, j] h[m, j]; k step ks covers, in lane l, columns lg*16 + 8 ks + 0..7
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
          xacc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
              af[b][ks], as_bf8(make_uint4(hw[4 * ks], hw[4 * ks + 1], hw[4 * ks + 2], hw[4 * ks + 3])), xacc, 0, 0, 0);
      }
      if (live) {  // lane l holds ρ = g*8 + (l/32)*4 + 0..3 in registers 4g..4g+3: one 16-byte store per g < R/8
        float* pp = swe.part + ((int64_t)(n0 >> 7) * M + m) * R + lg * 4;
#pragma unroll
        for (int g4 = 0; g4 < R / 8; ++g4)
          *reinterpret_cast<float4*>(pp + g4 * 8) =
              make_float4(xacc[4 * g4], xacc[4 * g4 + 1], xacc[4 * g4 + 2], xacc[4 * g4 + 3]);
      }
    }
    return;
  }

  if constexpr (kEpi == kEpiSwiGluBwd) {
    // SwiGLU backward (fused_mlp.py:112-175, the _bwd_kernel math) on dhm = bf16(acc), the reference's _scaled_mm
    // output.  The wave walks its 8 blocks of 32 x 32 (row block mt outer, column block nt inner); per block it
    // recomputes g, u, h from the saved gu, forms dh = bf16(dhm + dxd·A_dᵀ), du and dg, writes MX(dg) and MX(du)
    // into the dgrad GEMM's operand, and computes, as bwd_kernel does for one column tile of its quad:
    //   the dxa_g | dxa_u | xS_down products D[ρ][m] over the block's columns, added in registers over the tile's
    //   column blocks in order nt = 0..3 (bwd_kernel's fixed-order sum over the quad's waves: the partials are
    //   the same bits) and stored as the tile's partial after the row block's last column block;
    //   the dB_g, dB_u, dA_dᵀ contributions D[j][ρ] over the block's 32 rows (LDS transposes, 16x16x32 products),
    //   summed over the 4 waves in wave order and over the two row blocks in order, in LDS, and stored as the
    //   tile row's partial.
    // gu of the next block is loaded before the current block's stores, so waiting for it never waits for them
    // (the memory counter completes in order); the small per-row operands are loaded once per row block and the
    // weights are staged in LDS once per tile.
    constexpr int R = kR;
    static_assert(R == 16, "the backward epilogue's LDS is laid out for r = 16");
    const int lg = lane >> 5, rho = lane & 31;
    const int Tpad = (M + 127) / 128 * 128;  // rows of the transposed operands and of the scale buffer
    // dhm as packed bf16 pairs (columns lg*16 + 2k, +1 of each block): the fp32 accumulators are dead from here
    uint32_t dm[4][2][8];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt)
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          dm[nt][mt][k] = pack_bf16x2(acc[nt][mt][2 * k], acc[nt][mt][2 * k + 1]);
          // pin the packed value here: left alone, the compiler sinks each conversion to its block and keeps
          // all 128 fp32 accumulators live through the first blocks (and spills)
          asm volatile("" : "+v"(dm[nt][mt][k]));
        }
    // the ring is free once every wave's DMAs have landed (vmcnt(0) above) and its fragment reads are done
    lds_barrier();
    const uint32_t lw0 = lds0 + kBwdWOff;
    {  // the tile's weights into LDS: 6 arrays of 4 KB, 24 DMAs of 1 KB, 6 per wave (lane i lands at 16 i)
#pragma unroll
      for (int j = 0; j < 6; ++j) {
        const int i = wave * 6 + j, arr = i >> 2, k = i & 3;  // wave-uniform
        const uint16_t* src;
        if (arr < 3) {  // B_g, B_u, A_dᵀ rows n0 + (k*1024 + 16 lane) / 32: contiguous 4 KB
          const uint16_t* base = arr == 0 ? swb.bg : arr == 1 ? swb.bu : swb.adT;
          src = base + (int64_t)n0 * R + k * 512 + lane * 8;
        } else {  // B_gᵀ, B_uᵀ, A_d row ρ = 4 k + lane / 16, columns n0 + 8 (lane % 16) ..
          const uint16_t* base = arr == 3 ? swb.bgT : arr == 4 ? swb.buT : swb.ad;
          src = base + (int64_t)(4 * k + (lane >> 4)) * N + n0 + (lane & 15) * 8;
        }
        dma16(src, lw0 + arr * 4096 + k * 1024);
      }
    }
    const uint16_t* const wl = reinterpret_cast<const uint16_t*>(lds + kBwdWOff);
    uint16_t* const trw = reinterpret_cast<uint16_t*>(lds + wave * kBwdTrBytes);
    float* const dbx = reinterpret_cast<float*>(trw);  // the wave's dB exchange (after its transposes are read)
    float* const dbl = reinterpret_cast<float*>(lds + kBwdDbOff);
    auto fetch = [&](int b, uint32_t* w) {  // g | u of block b (nt = b % 4, mt = b / 4)
      const int mc = min(m0 + wm * 64 + (b >> 2) * 32 + (lane & 31), M - 1);
      const int c = n0 + (b & 3) * 32 + lg * 16;
      load16_rc(swb.gu, mc, c, 2 * N, true, w);
      load16_rc(swb.gu, mc, N + c, 2 * N, true, w + 8);
    };
    uint32_t gbuf[2][16];
    fetch(0, gbuf[0]);
    wait_vmcnt<4>();  // the weight DMAs, issued before the 4 loads of block 0's gu, have landed
    lds_barrier();
    v8bf xg, xu, xd, tg, tu, td;  // the row block's xs, dxd rows and their transposed forms
    float4 xa[3][2];              // dxa | dxa_u | xS_down of the row block, running over its column blocks
#pragma unroll
    for (int b = 0; b < 8; ++b) {
      const int nt = b & 3, mt = b >> 2;
      const int jb = n0 + nt * 32;
      const int rb = m0 + wm * 64 + mt * 32;
      const int m = rb + (lane & 31);
      const bool live = m < M;
      const int mc = live ? m : M - 1;
      __builtin_amdgcn_sched_barrier(0);  // blocks stay in order: only the explicit prefetch runs ahead
      if (b + 1 < 8) fetch(b + 1, gbuf[(b + 1) & 1]);
      if (nt == 0) {
        xg = load_bf8(swb.xs + (int64_t)mc * 2 * R + lg * 8);
        xu = load_bf8(swb.xs + (int64_t)mc * 2 * R + R + lg * 8);
        xd = load_bf8(swb.dxd + (int64_t)mc * R + lg * 8);
        const int rr = lane & 15, mo = min(rb, Tpad - 32) + (lane >> 4) * 8;  // rows past Tpad: any (they add 0)
        tg = load_bf8(swb.xsT + (int64_t)rr * Tpad + mo);
        tu = load_bf8(swb.xsT + (int64_t)(R + rr) * Tpad + mo);
        td = load_bf8(swb.dxdT + (int64_t)rr * Tpad + mo);
      }
      // Every block runs branch-free, also a block of rows past Tpad (in the last tile row only): its loads are
      // clamped to real rows, it stores nothing, and its zeroed values add nothing to the sums.  (Under a
      // branch the compiler's counter waits, merged over both paths, would also wait for the prefetch.)
      v4f dbg[2], dbu[2], dad[2];
      {
        uint32_t* gw = gbuf[b & 1];
        uint32_t* uw = gbuf[b & 1] + 8;
        // weights of these 32 columns from LDS: LoRA-B rows jb + pi_col(lane % 32) (B_g, B_u, A_dᵀ)
        const int wrow = (nt * 32 + pi_col(lane & 31)) * R + lg * 8;
        {
          const v16f d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*reinterpret_cast<const v8bf*>(wl + wrow), xg,
                                                                 v16f{}, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 16; i += 2) {
            float a = bf16_lo(gw[i / 2]) + swb.s_g * d[i], c = bf16_hi(gw[i / 2]) + swb.s_g * d[i + 1];
            gw[i / 2] = rnd2(a, c);
          }
        }
        {
          const v16f d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*reinterpret_cast<const v8bf*>(wl + 2048 + wrow),
                                                                 xu, v16f{}, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 16; i += 2) {
            float a = bf16_lo(uw[i / 2]) + swb.s_u * d[i], c = bf16_hi(uw[i / 2]) + swb.s_u * d[i + 1];
            uw[i / 2] = rnd2(a, c);
          }
        }
        uint32_t dp[8];
        {
          const v16f d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*reinterpret_cast<const v8bf*>(wl + 4096 + wrow),
                                                                 xd, v16f{}, 0, 0, 0);
#pragma unroll
          for (int i = 0; i < 16; i += 2) {
            float a = bf16_lo(dm[nt][mt][i / 2]) + d[i], c = bf16_hi(dm[nt][mt][i / 2]) + d[i + 1];
            dp[i / 2] = rnd2(a, c);  // dh
          }
        }
        uint32_t dgw[8], duw[8], hw[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float g0 = bf16_lo(gw[i]), g1 = bf16_hi(gw[i]);
          const float u0 = bf16_lo(uw[i]), u1 = bf16_hi(uw[i]);
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
        {  // MX(dg) at columns jb.., MX(du) at N + jb.. of the [*, 2N] operand: codes of live rows, scale bytes
           // of every row below Tpad (0 for padded rows)
          uint4 c;
          const uint32_t eg = quant16_codes(dgw, c);
          if (live) store_codes<MX_NT_FUSED>(swb.q + tiled_offset(m, jb + lg * 16, 2 * N), c);
          const uint32_t eu = quant16_codes(duw, c);
          if (live) store_codes<MX_NT_FUSED>(swb.q + tiled_offset(m, N + jb + lg * 16, 2 * N), c);
          if (lg == 0 && rb < Tpad) {
            store_scale<MX_NT_FUSED>(swb.s + blocked_offset(m, jb >> 5, 2 * N / 128), live ? (uint8_t)eg : (uint8_t)0);
            store_scale<MX_NT_FUSED>(swb.s + blocked_offset(m, (N + jb) >> 5, 2 * N / 128),
                                     live ? (uint8_t)eu : (uint8_t)0);
          }
        }
        if (!live) {  // padded rows add nothing to the sums below
#pragma unroll
          for (int i = 0; i < 8; ++i) dgw[i] = duw[i] = hw[i] = 0u;
        }
        // dxa_g | dxa_u | xS_down over this block's columns, D[ρ][m] (lane l: m = l % 32, ρ = (i / 4) * 8 +
        // (l / 32) * 4 + i % 4: registers 0..7 hold ρ < 16), with rows ρ of B_gᵀ, B_uᵀ, A_d (zero past r) at the
        // lane's columns as the first operand
#pragma unroll
        for (int p = 0; p < 3; ++p) {
          const uint32_t* w = p == 0 ? dgw : p == 1 ? duw : hw;
          v16f d = v16f{};
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            const v8bf f = *reinterpret_cast<const v8bf*>(wl + (3 + p) * 2048 + (rho & 15) * 128 + nt * 32 + lg * 16 +
                                                          8 * ks);
            d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                rho < R ? f : v8bf{}, as_bf8(make_uint4(w[4 * ks], w[4 * ks + 1], w[4 * ks + 2], w[4 * ks + 3])), d,
                0, 0, 0);
          }
          const float4 lo = make_float4(d[0], d[1], d[2], d[3]), hi = make_float4(d[4], d[5], d[6], d[7]);
          if (nt == 0) {
            xa[p][0] = lo;
            xa[p][1] = hi;
          } else {
            xa[p][0] = make_float4(xa[p][0].x + lo.x, xa[p][0].y + lo.y, xa[p][0].z + lo.z, xa[p][0].w + lo.w);
            xa[p][1] = make_float4(xa[p][1].x + hi.x, xa[p][1].y + hi.y, xa[p][1].z + hi.z, xa[p][1].w + hi.w);
          }
          if (nt == 3 && live) {  // the tile's partial: row m, columns p*R + g4*8 + (l/32)*4 + 0..3
            float* pp = swb.dxa + ((int64_t)(n0 >> 7) * M + m) * 3 * R + p * R + lg * 4;
            *reinterpret_cast<float4*>(pp) = xa[p][0];
            *reinterpret_cast<float4*>(pp + 8) = xa[p][1];
          }
        }
        // dB_g, dB_u, dA_dᵀ: D[j][ρ] = Σ_m dg[m, j] xs_g[m, ρ] etc. over the block's 32 rows
        tr_store(trw, lane, dgw);
        tr_store(trw + 32 * kTrLd, lane, duw);
        tr_store(trw + 64 * kTrLd, lane, hw);
#pragma unroll
        for (int jh = 0; jh < 2; ++jh) {
          dbg[jh] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(tr_operand(trw, jh * 16, lane), tg, v4f{}, 0, 0, 0);
          dbu[jh] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(tr_operand(trw + 32 * kTrLd, jh * 16, lane), tu, v4f{},
                                                            0, 0, 0);
          dad[jh] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(tr_operand(trw + 64 * kTrLd, jh * 16, lane), td, v4f{},
                                                            0, 0, 0);
        }
      }
      // the 4 waves' dB sums of this block, added in wave order: each wave puts its [3][32 x 16] floats in its
      // own transpose tiles (dB_g, dB_u as [j][ρ], dA_d as [ρ][j]), then
      // every thread adds one or two float4 of the four: into the tile's sums (first row block) or onto them and
      // into the tile row's partial (second row block)
#pragma unroll
      for (int jh = 0; jh < 2; ++jh) {
        const int j0 = jh * 16 + (lane >> 4) * 4, r0 = lane & 15;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          dbx[(j0 + i) * 16 + r0] = dbg[jh][i];
          dbx[512 + (j0 + i) * 16 + r0] = dbu[jh][i];
        }
        *reinterpret_cast<float4*>(dbx + 1024 + r0 * 32 + j0) =
            make_float4(dad[jh][0], dad[jh][1], dad[jh][2], dad[jh][3]);
      }
      lds_barrier();
      for (int f = tid; f < 384; f += 256) {  // 3 x 128 float4 per wave
        const int e = (f & 127) * 4, p = f >> 7;
        const float* base = reinterpret_cast<const float*>(lds) + p * 512 + e;
        float4 v = *reinterpret_cast<const float4*>(base);
#pragma unroll
        for (int w = 1; w < 4; ++w) {
          const float4 t = *reinterpret_cast<const float4*>(base + w * (kBwdTrBytes / 4));
          v = make_float4(v.x + t.x, v.y + t.y, v.z + t.z, v.w + t.w);
        }
        float4* acc_db = reinterpret_cast<float4*>(dbl + (nt * 3 + p) * 512 + e);
        if (mt == 0) {
          *acc_db = v;
        } else {
          const float4 a = *acc_db;
          v = make_float4(a.x + v.x, a.y + v.y, a.z + v.z, a.w + v.w);
          float* dst = p == 0   ? swb.dbg + ((int64_t)mt_ * N + jb + e / 16) * R + e % 16
                       : p == 1 ? swb.dbu + ((int64_t)mt_ * N + jb + e / 16) * R + e % 16
                                : swb.dad + ((int64_t)mt_ * R + e / 32) * N + jb + e % 32;
          *reinterpret_cast<float4*>(dst) = v;
        }
      }
      lds_barrier();
    }
    return;
  }

  // the output segment of this tile (wave-uniform)
  int sg = 0;
#pragma unroll
  for (int k = 1; k < 4; ++k)
    if (k < cseg.n && n0 >= cseg.col0[k]) sg = k;
  uint16_t* const C = cseg.ptr[sg];
  const int64_t ldc = cseg.ld[sg];
  const int ncol0 = cseg.col0[sg];
  const uint16_t* const lp = lora.p + cseg.rcol[sg];  // the segment's rank-r columns of P and Q
  const uint16_t* const lq = lora.q + cseg.rcol[sg];
  // epilogue: lane holds row m = m0 + wm*64 + mt*32 + lane%32 and columns n0 + wn*128 + nt*32 + g*8 +
  // (lane/32)*4 + 0..3 in acc[nt][mt][4g .. 4g+3]; with B in the pi_col order (b_pi) the 16 contiguous columns
  // n0 + wn*128 + nt*32 + (lane/32)*16 + i in acc[nt][mt][i].
  // The rank-r operands: the P rows of both row halves are loaded first, the Q rows of column block nt + 1 while
  // block nt is finished, so the wave waits for one memory latency, not one per 32 x 32 block.  Rounding to bf16
  // goes through v_cvt_pk_bf16_f32 (rnd2), pairwise.
  constexpr int kH = kR > 0 ? kR / 16 : 1;
  v8bf pf[2][kH], qf[2][kH];
  auto load_q = [&](int nt, v8bf* dst) {
    const int nr = min(n0 + wn * 128 + nt * 32 + (b_pi ? pi_col(lane & 31) : (lane & 31)), N - 1);
#pragma unroll
    for (int h = 0; h < kH; ++h)
      dst[h] = *reinterpret_cast<const v8bf*>(lq + (int64_t)nr * lora.ld_q + h * 16 + (lane >> 5) * 8);
  };
  if constexpr (kR > 0) {
    bool p_ready = true;  // P summed in this launch: its rows published, or this tile sums them (presum_device.h)
    if constexpr (kFoldSum<kR, kNW, kEpi>) {
      if (pre.blocks) p_ready = presum_wait(pre, m0, min(m0 + kBM, M), &arrived);
    }
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int mc = min(m0 + wm * 64 + mt * 32 + (lane & 31), M - 1);
#pragma unroll
      for (int h = 0; h < kH; ++h) {
        if constexpr (kFoldSum<kR, kNW, kEpi>) {
          if (pre.blocks) {
            pf[mt][h] = p_ready ? presum_load8(lp + (int64_t)mc * lora.ld_p + h * 16 + (lane >> 5) * 8)
                                : presum_row8(pre, mc, h * 16 + (lane >> 5) * 8, kR);
            continue;
          }
        }
        pf[mt][h] = *reinterpret_cast<const v8bf*>(lp + (int64_t)mc * lora.ld_p + h * 16 + (lane >> 5) * 8);
      }
    }
    load_q(0, qf[0]);
  }
#pragma unroll
  for (int nt = 0; nt < 4; ++nt) {
    const int nb = n0 + wn * 128 + nt * 32;
    if constexpr (kR > 0) {
      if (nt + 1 < 4) load_q(nt + 1, qf[(nt + 1) & 1]);
    }
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int m = m0 + wm * 64 + mt * 32 + (lane & 31);
      const v16f o = acc[nt][mt];
      uint32_t wv[8];  // packed bf16 pairs of o[2k], o[2k + 1]
      if constexpr (kR > 0) {
        v16f l = v16f{};
#pragma unroll
        for (int h = 0; h < kH; ++h) l = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qf[nt & 1][h], pf[mt][h], l, 0, 0, 0);
#pragma unroll
        for (int k = 0; k < 8; ++k) {  // bf16(bf16(acc) + alpha · P·Qᵀ)
          float a = o[2 * k], b = o[2 * k + 1];
          rnd2(a, b);
          a += lora.alpha * l[2 * k];
          b += lora.alpha * l[2 * k + 1];
          wv[k] = rnd2(a, b);
        }
      } else {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          float a = o[2 * k], b = o[2 * k + 1];
          wv[k] = rnd2(a, b);
        }
      }
      if (m >= M) continue;
      if (b_pi) {  // columns nb + (lane/32)*16 + 0..15 (N % 128 == 0: all inside)
        const int n = nb + (lane >> 5) * 16;
        if (c_ft) {
          uint16_t* p = C + ft_offset(m, n, N);
          *reinterpret_cast<uint4*>(p) = make_uint4(wv[0], wv[1], wv[2], wv[3]);
          *reinterpret_cast<uint4*>(p + 512) = make_uint4(wv[4], wv[5], wv[6], wv[7]);
        } else {
          uint16_t* p = C + (int64_t)m * ldc + (n - ncol0);
          *reinterpret_cast<uint4*>(p) = make_uint4(wv[0], wv[1], wv[2], wv[3]);
          *reinterpret_cast<uint4*>(p + 8) = make_uint4(wv[4], wv[5], wv[6], wv[7]);
        }
        continue;
      }
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = nb + g * 8 + (lane >> 5) * 4;
        if (n < N)
          *reinterpret_cast<uint2*>(C + (c_ft ? ft_offset(m, n, N) : (int64_t)m * ldc + (n - ncol0))) =
              make_uint2(wv[2 * g], wv[2 * g + 1]);
      }
    }
  }
}

int cached_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cus[dev]) {
    int v = 0;
    if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
    cus[dev] = v;
  }
  return cus[dev];
}

// Split the tail wave along K when it would leave more than half of the workgroup slots idle (slots = CUs x
// workgroups per CU: the LDS ring takes 136 KB at kNW = 2, 78 KB at kNW = 1).  Returns the workspace bytes
// the plan needs (0 without a split).
template <int kNW>
int64_t make_plan(int64_t M, int64_t N, int64_t K, int cus, Plan& p) {
  using S = Shape<kNW>;
  const int slots = cus * (kNW == 2 ? 1 : 2);
  p.tm = (int)((M + kBM - 1) / kBM);
  p.tn = (int)((N + S::kBN - 1) / S::kBN);
  const int total = p.tm * p.tn, ns = (int)(K / kBK);
  const int rem = total % slots;
  p.full = total;
  p.nsplit = 0;
  p.parts = 1;
  p.chunk = ns;
  // Two co-resident workgroups per CU already overlap one tile's pipeline fill and epilogue with the other's
  // main loop; splitting the tail along K measured slower there (down: 184-199 us split vs 143-149 whole).
  if (kNW == 2 && rem > 0 && 2 * rem <= slots && rem <= kMaxSplitTiles) {
    int parts = min(kMaxParts, slots / rem);
    int chunk = 2 * ((ns + 2 * parts - 1) / (2 * parts));
    parts = (ns + chunk - 1) / chunk;
    if (parts >= 2 && chunk >= 4) {
      p.full = total - rem;
      p.nsplit = rem;
      p.parts = parts;
      p.chunk = chunk;
    }
  }
  p.per_full = (p.full + 7) / 8;
  p.per_split = (p.nsplit * p.parts + 7) / 8;
  if (!p.nsplit) return 0;
  return kCounterBytes + (int64_t)p.nsplit * p.parts * S::kPartBytes;
}

template <int kNW>
void launch(const uint8_t* A, const uint8_t* SA, int64_t lda, const uint8_t* B, const uint8_t* SB, int64_t ldb,
            int M, int N, int K, const CSeg& cseg, const Lora& lo, int r, const Plan& plan, int layout,
            const TnBatch& tnb, int64_t tn_blocks, const PreSum& pre, hipStream_t stm) {
  using S = Shape<kNW>;
  dim3 grid((unsigned)(pre.blocks + 8 * plan.per_full + 8 * plan.per_split + tn_blocks));
#define GEMM_ARGS A, SA, lda, B, SB, ldb, M, N, K, cseg, lo, plan, layout, SwEpi{}, SwBwd{}, tnb, pre
  if (!lo.p) gemm_kernel<0, kNW, kEpiPlain><<<grid, S::kThreads, 0, stm>>>(GEMM_ARGS);
  else if (r == 16) gemm_kernel<16, kNW, kEpiPlain><<<grid, S::kThreads, 0, stm>>>(GEMM_ARGS);
  else if (r == 32) gemm_kernel<32, kNW, kEpiPlain><<<grid, S::kThreads, 0, stm>>>(GEMM_ARGS);
  else if (r == 48) gemm_kernel<48, kNW, kEpiPlain><<<grid, S::kThreads, 0, stm>>>(GEMM_ARGS);
  else gemm_kernel<64, kNW, kEpiPlain><<<grid, S::kThreads, 0, stm>>>(GEMM_ARGS);
#undef GEMM_ARGS
}

}  // namespace

extern "C" int64_t mxfp8_gemm_workspace_size(int64_t M, int64_t N, int64_t K) {
  if (M <= 0 || N <= 0 || K <= 0 || K % 128 || N % 128) return 0;
  Plan p;
  return make_plan<2>(M, N, K, cached_cus(), p);  // only the 8-wave shape splits
}

namespace {

int gemm_impl(const void* a, const void* sa, int64_t lda, const void* b, const void* sb, int64_t ldb, int64_t M,
              int64_t N, int64_t K, CSeg cseg, const void* lora_p, int64_t ld_p, const void* lora_q, int64_t ld_q,
              int64_t r, float alpha, int64_t layout, void* workspace, int64_t workspace_bytes, void* stream,
              const TnBatch& tnb = TnBatch{}, int64_t tn_blocks = 0, const PreSum& pre = PreSum{}) {
  void* const c = cseg.ptr[0];
  int64_t ldc = cseg.ld[0];
  MX_CHECK_ARG(a && sa && b && sb && c, "mxfp8_gemm_nt: null pointer");
  MX_CHECK_ARG(M >= 0 && N > 0 && K > 0 && K % 128 == 0 && N % 128 == 0,
               "mxfp8_gemm_nt: need K %% 128 == 0 and N %% 128 == 0 (M=%lld N=%lld K=%lld)", (long long)M,
               (long long)N, (long long)K);
  MX_CHECK_ARG(M < (1LL << 30) && N < (1LL << 30) && K < (1LL << 30), "mxfp8_gemm_nt: dimension too large");
  MX_CHECK_ARG(layout >= 0 && layout <= 31,
               "mxfp8_gemm_nt: layout must be 0..31 (bit 0: A MX-tiled, bit 1: B MX-tiled, bit 2: 8-wave shape, "
               "bit 3: C in the FT layout, bit 4: B rows in the pi_col order)");
  if (layout & 1) lda = K;  // the tiled layouts have no row stride
  if (layout & 2) ldb = K;
  if (layout & MXFP8_GEMM_C_FT) ldc = N;
  const int64_t seg_w0 = cseg.n > 1 ? cseg.col0[1] : N;  // width of the first segment
  MX_CHECK_ARG(lda >= K && ldb >= K && lda % 16 == 0 && ldb % 16 == 0 && ldc >= seg_w0 && ldc % 4 == 0,
               "mxfp8_gemm_nt: bad strides");
  cseg.ld[0] = ldc;
  MX_CHECK_ARG(256LL * lda < (1LL << 32) && 256LL * ldb < (1LL << 32), "mxfp8_gemm_nt: stride too large");
  MX_CHECK_ARG(mx_aligned(a, 16) && mx_aligned(b, 16) && mx_aligned(sa, 16) && mx_aligned(sb, 16) &&
                   mx_aligned(c, 8),
               "mxfp8_gemm_nt: misaligned buffer");
  MX_CHECK_ARG(!(layout & MXFP8_GEMM_B_PI) || (mx_aligned(c, 16) && ((layout & MXFP8_GEMM_C_FT) || ldc % 8 == 0)),
               "mxfp8_gemm_nt: MXFP8_GEMM_B_PI stores 16-byte pieces (C 16-byte aligned, ldc %% 8 == 0)");
  MX_CHECK_ARG(workspace_bytes >= 0 && (workspace_bytes == 0 || (workspace && mx_aligned(workspace, 256))),
               "mxfp8_gemm_nt: workspace must be 256-byte aligned");
  if (lora_p) {
    MX_CHECK_ARG(lora_q && (r == 16 || r == 32 || r == 48 || r == 64),
                 "mxfp8_gemm_nt: epilogue needs P, Q and r in {16, 32, 48, 64}");
    MX_CHECK_ARG(ld_p >= r && ld_q >= r && ld_p % 8 == 0 && ld_q % 8 == 0 && mx_aligned(lora_p, 16) &&
                     mx_aligned(lora_q, 16),
                 "mxfp8_gemm_nt: bad epilogue strides/alignment");
  }
  if (M == 0) return MXFP8_OK;
  Plan plan;
  const bool wide = layout & MXFP8_GEMM_WIDE;
  const int64_t need = wide ? make_plan<2>(M, N, K, cached_cus(), plan) : make_plan<1>(M, N, K, cached_cus(), plan);
  if (need > workspace_bytes) {  // no (or too small a) workspace: run every tile whole
    plan.full = plan.tm * plan.tn;
    plan.per_full = (plan.full + 7) / 8;
    plan.nsplit = 0;
    plan.per_split = 0;
    plan.parts = 1;
  }
  plan.cnt = plan.nsplit ? (int*)workspace : nullptr;
  plan.ws = plan.nsplit ? (float4*)((char*)workspace + kCounterBytes) : nullptr;
  Lora lo{(const uint16_t*)lora_p, ld_p, (const uint16_t*)lora_q, ld_q, alpha};
  const uint8_t *A = (const uint8_t*)a, *SA = (const uint8_t*)sa, *B = (const uint8_t*)b, *SB = (const uint8_t*)sb;
  const int tiled = (int)(layout & ~MXFP8_GEMM_WIDE);
  if (wide)
    launch<2>(A, SA, lda, B, SB, ldb, (int)M, (int)N, (int)K, cseg, lo, (int)r, plan, tiled, tnb, 0, PreSum{},
              (hipStream_t)stream);
  else
    launch<1>(A, SA, lda, B, SB, ldb, (int)M, (int)N, (int)K, cseg, lo, (int)r, plan, tiled, tnb, tn_blocks, pre,
              (hipStream_t)stream);
  MX_CHECK_LAUNCH("mxfp8_gemm_nt");
  return MXFP8_OK;
}

}  // namespace

extern "C" int mxfp8_gemm_nt(const void* a, const void* sa, int64_t lda, const void* b, const void* sb, int64_t ldb,
                             int64_t M, int64_t N, int64_t K, void* c, int64_t ldc, const void* lora_p, int64_t ld_p,
                             const void* lora_q, int64_t ld_q, int64_t r, float alpha, int64_t layout,
                             void* workspace, int64_t workspace_bytes, void* stream) {
  CSeg cs{};
  cs.n = 1;
  cs.ptr[0] = (uint16_t*)c;
  cs.ld[0] = ldc;
  return gemm_impl(a, sa, lda, b, sb, ldb, M, N, K, cs, lora_p, ld_p, lora_q, ld_q, r, alpha, layout, workspace,
                   workspace_bytes, stream);
}

extern "C" int mxfp8_gemm_nt_tn(const void* a, const void* sa, int64_t lda, const void* b, const void* sb,
                                int64_t ldb, int64_t M, int64_t N, int64_t K, void* c, int64_t ldc, const void* lora_p,
                                int64_t ld_p, const void* lora_q, int64_t ld_q, int64_t r, float alpha, int64_t layout,
                                const mxfp8_lora_tn_job* jobs, int64_t n_jobs, int64_t T_tn, int64_t K_tn,
                                int64_t chunks, float* part, void* stream) {
  MX_CHECK_ARG(M > 0 && lora_p && (r == 16 || r == 32 || r == 48) && !(layout & MXFP8_GEMM_WIDE),
               "mxfp8_gemm_nt_tn: needs M > 0, a rank-16, 32 or 48 LoRA epilogue and the 4-wave shape (r=%lld "
               "layout=%lld)",
               (long long)r, (long long)layout);
  TnBatch tnb;
  TnSumBatch sa_tn;
  int64_t nb = 0, ns = 0;
  int rc = tn_batch_tables("mxfp8_gemm_nt_tn", jobs, n_jobs, T_tn, K_tn, chunks, part, tnb, sa_tn, nb, ns);
  if (rc != MXFP8_OK) return rc;
  MX_CHECK_ARG(nb + (M + kBM - 1) / kBM * (N / 128) + 8 < (1LL << 31), "mxfp8_gemm_nt_tn: too many workgroups");
  CSeg cs{};
  cs.n = 1;
  cs.ptr[0] = (uint16_t*)c;
  cs.ld[0] = ldc;
  rc = gemm_impl(a, sa, lda, b, sb, ldb, M, N, K, cs, lora_p, ld_p, lora_q, ld_q, r, alpha, layout, nullptr, 0, stream,
                 tnb, nb);
  if (rc != MXFP8_OK) return rc;
  return tn_sum_batch_launch(sa_tn, ns, (hipStream_t)stream, "mxfp8_gemm_nt_tn");
}

// ------------------------------------------------------------------ the epilogue operand summed in the launch
// The publication flags of mxfp8_gemm_nt_sum's summing workgroups: one file-scope device array per GPU, held
// until the process ends.  Host code uses its device address (hipGetSymbolAddress, looked up once per device with
// that device current), never the array's name.  Flags hold launch ids, unique per process, so they need no
// clearing.  Each launch takes its own slice of the array, the slice after the previous launch's, so launches
// that overlap on one GPU (other streams) use different flags unless more than the array's worth of blocks is in
// flight; if they do collide, a tile sums its rows itself after its polls run out (same results, slower).
constexpr int64_t kPreSumMaxBlocks = 1 << 16;
static __device__ __align__(256) unsigned long long presum_flags[kPreSumMaxBlocks];

namespace {

constexpr int kMaxDevices = 64;
std::mutex presum_mu;
unsigned long long* presum_flags_dev[kMaxDevices] = {};
std::atomic<unsigned long long> presum_next_id{1};

unsigned long long* presum_flags_on_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    mxabi::set_error("mxfp8_gemm_nt_sum: no current device (or device index >= %d)", kMaxDevices);
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(presum_mu);
  if (!presum_flags_dev[dev]) {
    void* ptr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(presum_flags));
    if (e != hipSuccess || !ptr) {
      mxabi::set_error("mxfp8_gemm_nt_sum: hipGetSymbolAddress(presum_flags) failed on device %d: %s", dev,
                       hipGetErrorString(e));
      return nullptr;
    }
    presum_flags_dev[dev] = static_cast<unsigned long long*>(ptr);
  }
  return presum_flags_dev[dev];
}

}  // namespace

extern "C" int mxfp8_gemm_nt_sum(const void* a, const void* sa, int64_t lda, const void* b, const void* sb,
                                 int64_t ldb, int64_t M, int64_t N, int64_t K, void* c, int64_t ldc,
                                 const float* part, int64_t n_parts, float part_scale, void* lora_p,
                                 const void* lora_q, int64_t ld_q, int64_t r, float alpha, int64_t layout,
                                 int64_t wait_limit, void* stream) {
  MX_CHECK_ARG(M > 0 && part && lora_p && lora_q && r == 16 && !(layout & MXFP8_GEMM_WIDE) && n_parts >= 1,
               "mxfp8_gemm_nt_sum: needs M > 0, partials, P and Q, r == 16 and the 4-wave shape (r=%lld layout=%lld)",
               (long long)r, (long long)layout);
  MX_CHECK_ARG(mx_aligned(part, 16) && mx_aligned(lora_p, 16), "mxfp8_gemm_nt_sum: misaligned part or P");
  const int64_t count4 = M * r / 4;
  const int64_t blocks = ((count4 + 255) / 256 + 7) / 8 * 8;
  MX_CHECK_ARG(blocks <= kPreSumMaxBlocks && n_parts < (1LL << 31), "mxfp8_gemm_nt_sum: M * r = %lld beyond %lld",
               (long long)(M * r), (long long)(kPreSumMaxBlocks * 1024));
  CSeg cs{};
  cs.n = 1;
  cs.ptr[0] = (uint16_t*)c;
  cs.ld[0] = ldc;
  // A launch captured into a graph would keep its launch id on every replay: a tile of the second replay could
  // find its flags already holding that id from the first and read P before this replay's sums.  A captured call
  // (or one on a stream whose capture state cannot be read) therefore sums P in a launch of its own, the same
  // bits, before the plain GEMM.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing((hipStream_t)stream, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) {
    const int rc = mxfp8_sum_parts(part, n_parts, M * r, part_scale, lora_p, 1, stream);
    if (rc != MXFP8_OK) return rc;
    return gemm_impl(a, sa, lda, b, sb, ldb, M, N, K, cs, lora_p, r, lora_q, ld_q, r, alpha, layout, nullptr, 0,
                     stream);
  }
  unsigned long long* flags = presum_flags_on_current_device();
  if (!flags) return MXFP8_ERR_ARG;
  PreSum pre{};
  pre.part = part;
  pre.out = (uint16_t*)lora_p;
  pre.id = presum_next_id.fetch_add(1);
  pre.flags = flags + (int64_t)((pre.id * (unsigned long long)blocks) % (unsigned long long)(kPreSumMaxBlocks - blocks + 1));
  pre.count4 = count4;
  pre.n_parts = (int)n_parts;
  pre.blocks = (int)blocks;
  pre.rows_per_block = (int)(1024 / r);
  // polls of about 0.1 us each (s_sleep 2) before a tile sums its own rows: ~0.1 s by default, far beyond the
  // sums' own time
  pre.wait_limit = wait_limit < 0 ? (1 << 20) : (int)std::min<int64_t>(wait_limit, 1 << 30);
  pre.scale = part_scale;
  return gemm_impl(a, sa, lda, b, sb, ldb, M, N, K, cs, lora_p, r, lora_q, ld_q, r, alpha, layout, nullptr, 0, stream,
                   TnBatch{}, 0, pre);
}

extern "C" int mxfp8_gemm_nt_seg(const void* a, const void* sa, int64_t lda, const void* b, const void* sb,
                                 int64_t ldb, int64_t M, int64_t N, int64_t K, int64_t n_seg, const int64_t* seg_col0,
                                 void* const* seg_c, const int64_t* seg_ldc, const void* lora_p, int64_t ld_p,
                                 const void* lora_q, int64_t ld_q, int64_t r, const int64_t* seg_rcol, float alpha,
                                 int64_t layout, void* stream) {
  MX_CHECK_ARG(n_seg >= 1 && n_seg <= 4 && seg_col0 && seg_c && seg_ldc, "mxfp8_gemm_nt_seg: 1 to 4 segments");
  MX_CHECK_ARG(!(layout & (MXFP8_GEMM_WIDE | MXFP8_GEMM_C_FT | MXFP8_GEMM_B_PI)),
               "mxfp8_gemm_nt_seg: segments take the 4-wave shape, row-major C and B in row order");
  CSeg cs{};
  cs.n = (int)n_seg;
  for (int64_t k = 0; k < n_seg; ++k) {
    const int64_t c0 = seg_col0[k], c1 = k + 1 < n_seg ? seg_col0[k + 1] : N;
    MX_CHECK_ARG(seg_c[k] && c0 % 128 == 0 && c1 > c0 && c1 <= N && (k > 0 || c0 == 0) && seg_ldc[k] >= c1 - c0 &&
                     seg_ldc[k] % 4 == 0 && mx_aligned(seg_c[k], 8),
                 "mxfp8_gemm_nt_seg: segment %lld: columns from 0, increasing multiples of 128, ldc >= width",
                 (long long)k);
    cs.col0[k] = (int)c0;
    cs.ptr[k] = (uint16_t*)seg_c[k];
    cs.ld[k] = seg_ldc[k];
    if (seg_rcol && lora_p) {
      MX_CHECK_ARG(seg_rcol[k] >= 0 && seg_rcol[k] % 8 == 0 && seg_rcol[k] + r <= ld_p && seg_rcol[k] + r <= ld_q,
                   "mxfp8_gemm_nt_seg: segment %lld: rank columns must be a multiple of 8 within ld_p and ld_q",
                   (long long)k);
      cs.rcol[k] = (int)seg_rcol[k];
    }
  }
  return gemm_impl(a, sa, lda, b, sb, ldb, M, N, K, cs, lora_p, ld_p, lora_q, ld_q, r, alpha, layout, nullptr, 0,
                   stream);
}

extern "C" int mxfp8_gemm_swiglu_fwd(const void* a, const void* sa, const void* b, const void* sb, int64_t M, int64_t N,
                                     int64_t K, const void* xs, const void* bg, const void* bu, const void* ad,
                                     int64_t r, float s_g, float s_u, void* gu, void* q_h, void* s_h, float* part,
                                     void* stream) {
  MX_CHECK_ARG(a && sa && b && sb && xs && bg && bu && ad && gu && q_h && s_h && part,
               "mxfp8_gemm_swiglu_fwd: null pointer");
  MX_CHECK_ARG(M > 0 && N > 0 && K > 0 && N % 128 == 0 && K % 128 == 0 && (r == 16 || r == 32),
               "mxfp8_gemm_swiglu_fwd: need N %% 128 == 0, K %% 128 == 0, r in {16, 32} (M=%lld N=%lld K=%lld r=%lld)",
               (long long)M, (long long)N, (long long)K, (long long)r);
  MX_CHECK_ARG(M < (1LL << 30) && M * 2 * N < (1LL << 31) && K < (1LL << 24),
               "mxfp8_gemm_swiglu_fwd: M * 2N must stay below 2^31");
  MX_CHECK_ARG(mx_aligned(a, 16) && mx_aligned(b, 16) && mx_aligned(sa, 16) && mx_aligned(sb, 16) &&
                   mx_aligned(xs, 16) && mx_aligned(bg, 16) && mx_aligned(bu, 16) && mx_aligned(ad, 16) &&
                   mx_aligned(gu, 16) && mx_aligned(q_h, 16) && mx_aligned(part, 16),
               "mxfp8_gemm_swiglu_fwd: misaligned buffer");
  Plan plan;
  make_plan<1>(M, 2 * N, K, cached_cus(), plan);
  SwEpi sw{(const uint16_t*)xs, (const uint16_t*)bg, (const uint16_t*)bu, (const uint16_t*)ad, s_g, s_u,
           (uint16_t*)gu, (uint8_t*)q_h, (uint8_t*)s_h, part, (int)N};
  CSeg cs{};
  cs.n = 1;
  const dim3 grid((unsigned)(8 * plan.per_full));
  const int tiled = MXFP8_GEMM_A_TILED | MXFP8_GEMM_B_TILED;
  hipStream_t stm = (hipStream_t)stream;
  const uint8_t *A = (const uint8_t*)a, *SA = (const uint8_t*)sa, *B = (const uint8_t*)b, *SB = (const uint8_t*)sb;
  if (r == 16)
    gemm_kernel<16, 1, kEpiSwiGluFwd><<<grid, Shape<1>::kThreads, 0, stm>>>(
        A, SA, K, B, SB, K, (int)M, (int)(2 * N), (int)K, cs, Lora{}, plan, tiled, sw, SwBwd{}, TnBatch{}, PreSum{});
  else
    gemm_kernel<32, 1, kEpiSwiGluFwd><<<grid, Shape<1>::kThreads, 0, stm>>>(
        A, SA, K, B, SB, K, (int)M, (int)(2 * N), (int)K, cs, Lora{}, plan, tiled, sw, SwBwd{}, TnBatch{}, PreSum{});
  MX_CHECK_LAUNCH("mxfp8_gemm_swiglu_fwd");
  return MXFP8_OK;
}

extern "C" int mxfp8_gemm_swiglu_bwd(const void* a, const void* sa, const void* b, const void* sb, int64_t M, int64_t N,
                                     int64_t K, const void* gu, const void* xs, const void* xsT, const void* dxd,
                                     const void* dxdT, const void* bg, const void* bgT, const void* bu, const void* buT,
                                     const void* ad, const void* adT, int64_t r, float s_g, float s_u, void* q,
                                     void* s, float* dxa_part, float* dbg_part, float* dbu_part, float* dad_part,
                                     void* stream) {
  MX_CHECK_ARG(a && sa && b && sb && gu && xs && xsT && dxd && dxdT && bg && bgT && bu && buT && ad && adT && q && s &&
                   dxa_part && dbg_part && dbu_part && dad_part,
               "mxfp8_gemm_swiglu_bwd: null pointer");
  MX_CHECK_ARG(M > 0 && N > 0 && K > 0 && N % 128 == 0 && K % 128 == 0 && r == 16,
               "mxfp8_gemm_swiglu_bwd: need N %% 128 == 0, K %% 128 == 0, r == 16 (M=%lld N=%lld K=%lld r=%lld)",
               (long long)M, (long long)N, (long long)K, (long long)r);
  MX_CHECK_ARG(M < (1LL << 30) && M * 2 * N < (1LL << 31) && K < (1LL << 24),
               "mxfp8_gemm_swiglu_bwd: M * 2N must stay below 2^31");
  MX_CHECK_ARG(mx_aligned(a, 16) && mx_aligned(b, 16) && mx_aligned(sa, 16) && mx_aligned(sb, 16) &&
                   mx_aligned(gu, 16) && mx_aligned(xs, 16) && mx_aligned(xsT, 16) && mx_aligned(dxd, 16) &&
                   mx_aligned(dxdT, 16) && mx_aligned(bg, 16) && mx_aligned(bgT, 16) && mx_aligned(bu, 16) &&
                   mx_aligned(buT, 16) && mx_aligned(ad, 16) && mx_aligned(adT, 16) && mx_aligned(q, 16) &&
                   mx_aligned(dxa_part, 16) && mx_aligned(dbg_part, 16) && mx_aligned(dbu_part, 16) &&
                   mx_aligned(dad_part, 16),
               "mxfp8_gemm_swiglu_bwd: misaligned buffer");
  Plan plan;
  make_plan<1>(M, N, K, cached_cus(), plan);
  SwBwd sw{(const uint16_t*)gu,  (const uint16_t*)xs,  (const uint16_t*)xsT, (const uint16_t*)dxd,
           (const uint16_t*)dxdT, (const uint16_t*)bg, (const uint16_t*)bgT, (const uint16_t*)bu,
           (const uint16_t*)buT, (const uint16_t*)ad,  (const uint16_t*)adT, s_g, s_u, (uint8_t*)q, (uint8_t*)s,
           dxa_part, dbg_part, dbu_part, dad_part};
  CSeg cs{};
  cs.n = 1;
  const dim3 grid((unsigned)(8 * plan.per_full));
  const int tiled = MXFP8_GEMM_A_TILED | MXFP8_GEMM_B_TILED;
  gemm_kernel<16, 1, kEpiSwiGluBwd><<<grid, Shape<1>::kThreads, 0, (hipStream_t)stream>>>(
      (const uint8_t*)a, (const uint8_t*)sa, K, (const uint8_t*)b, (const uint8_t*)sb, K, (int)M, (int)N, (int)K, cs,
      Lora{}, plan, tiled, SwEpi{}, sw, TnBatch{}, PreSum{});
  MX_CHECK_LAUNCH("mxfp8_gemm_swiglu_bwd");
  return MXFP8_OK;
}
