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

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int tile_col(int i, int lane) { return (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3); }

typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef float v2f __attribute__((ext_vector_type(2)));

// Round a pair to bf16 with v_cvt_pk_bf16_f32 (round to nearest even, verified bit-exact against a software
// RNE on the device); returns the packed pair and leaves the bf16-valued floats in a, b.
__device__ __forceinline__ uint32_t rnd2(float& a, float& b) {
  const v2f f = {a, b};
  const uint32_t w = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, v2bf));
  a = __uint_as_float(w << 16);
  b = __uint_as_float(w & 0xffff0000u);
  return w;
}

// sigmoid(g) = 1 / (1 + exp(-g)) with the hardware exp2 and reciprocal (about 1 ulp each; the reference's
// Triton fp32 division is approximate as well); silu(g) = g * sigmoid(g).  exp(-g) overflowing to +inf
// gives sigmoid 0 and silu -0, as g / (exp(-g) + 1) does.
__device__ __forceinline__ float fast_sigmoid(float g) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.4426950408889634f));
}

__device__ __forceinline__ v8bf as_bf8(uint4 u) {
  u32x4 v = {u.x, u.y, u.z, u.w};
  return __builtin_bit_cast(v8bf, v);
}

__device__ __forceinline__ v8bf load_bf8(const uint16_t* p) { return as_bf8(*reinterpret_cast<const uint4*>(p)); }

// 8 bf16 of row `p` at columns base + {lg*4 + 0..3} and base + 8 + {lg*4 + 0..3} (one k-step of the permuted
// column order; lg = lane / 32)
__device__ __forceinline__ v8bf load_bf8_perm(const uint16_t* p, int base, int lg) {
  uint2 a = *reinterpret_cast<const uint2*>(p + base + lg * 4);
  uint2 b = *reinterpret_cast<const uint2*>(p + base + 8 + lg * 4);
  return as_bf8(make_uint4(a.x, a.y, b.x, b.y));
}

// registers 8s..8s+7 of a bf16-valued element tile as an MFMA operand
__device__ __forceinline__ v8bf regs_bf8(const float* v) {
  uint4 u;
  u.x = (__float_as_uint(v[0]) >> 16) | (__float_as_uint(v[1]) & 0xffff0000u);
  u.y = (__float_as_uint(v[2]) >> 16) | (__float_as_uint(v[3]) & 0xffff0000u);
  u.z = (__float_as_uint(v[4]) >> 16) | (__float_as_uint(v[5]) & 0xffff0000u);
  u.w = (__float_as_uint(v[6]) >> 16) | (__float_as_uint(v[7]) & 0xffff0000u);
  return as_bf8(u);
}

// 16 bf16 of the lane's row at columns jb + tile_col(i): four 8-byte loads, zeros for rows past the end
__device__ __forceinline__ void load_tile(const uint16_t* row, int jb, int lane, bool valid, float* v) {
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    uint2 w = valid ? *reinterpret_cast<const uint2*>(row + jb + g * 8 + (lane >> 5) * 4) : make_uint2(0, 0);
    v[4 * g + 0] = bf16_lo(w.x);
    v[4 * g + 1] = bf16_hi(w.x);
    v[4 * g + 2] = bf16_lo(w.y);
    v[4 * g + 3] = bf16_hi(w.y);
  }
}

// D[j][m] = Σ_ρ W[j, ρ] · X[m, ρ] for the 32 x 32 tile (W rows jb.., X rows of this lane), r in {16, 32}
template <int R>
__device__ __forceinline__ v16f lora_tile(const uint16_t* wrow, const v8bf* xf) {
  v16f d = v16f{};
#pragma unroll
  for (int h = 0; h < R / 16; ++h) d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(load_bf8(wrow + h * 16), xf[h], d, 0, 0, 0);
  return d;
}

// Quantize one 32-column block of the lane's row held as 8 packed bf16 pairs w[0..7] (columns
// tile_col(2k), tile_col(2k+1)) plus the other 16 values in lane ^ 32: codes of row mc, columns jb..jb+31
// (4-byte pieces) into q, row-major with Kq codes per row or MX-tiled (tiled_offset) with Kq codes per row;
// scale byte into the blocked layout (lanes < 32), or scale 0 for padded rows.
__device__ __forceinline__ void quant_tile(const uint32_t* w, int lane, int m, bool live, uint8_t* q, int64_t mc,
                                           int64_t Kq, bool tiled, int jb, uint8_t* s, int64_t s_col_tiles) {
  u16x2 mm = {0, 0};
#pragma unroll
  for (int k = 0; k < 8; ++k) mm = absmax2(mm, w[k]);
  uint32_t am = amax_bits(mm);
  am = max(am, (uint32_t)__shfl_xor((int)am, 32));
  const uint32_t e = e8m0_from_amax_bits(am);
  uint32_t c[4];
#pragma unroll
  for (int g = 0; g < 4; ++g) c[g] = encode4_bf16(w[2 * g], w[2 * g + 1], e);
  if (live) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int64_t k = jb + g * 8 + (lane >> 5) * 4;
      *reinterpret_cast<uint32_t*>(q + (tiled ? tiled_offset(mc, k, Kq) : mc * Kq + k)) = c[g];
    }
  }
  if (lane < 32) s[blocked_offset(m, jb >> 5, s_col_tiles)] = live ? (uint8_t)e : (uint8_t)0;
}

// registers 8s..8s+7 of an element tile held as packed words w[4s..4s+3], as an MFMA operand
__device__ __forceinline__ v8bf words_bf8(const uint32_t* w) { return as_bf8(make_uint4(w[0], w[1], w[2], w[3])); }

// ---------------------------------------------------------------------------------------------- forward
// grid (row blocks of 32 up to Tpad, column groups); 4 waves share the row block, wave w takes the group's
// column tiles w, w+4, ...; xS_down partial summed over the 4 waves in LDS (fixed order).
template <int R, bool kWriteQ>
__global__ __launch_bounds__(256) void fwd_kernel(const uint16_t* __restrict__ gu, const uint16_t* __restrict__ xs,
                                                  const uint16_t* __restrict__ bg, const uint16_t* __restrict__ bu,
                                                  const uint16_t* __restrict__ ad, int T, int N, int tiles_per_group,
                                                  float s_g, float s_u, uint8_t* __restrict__ q,
                                                  uint8_t* __restrict__ s, float* __restrict__ part,
                                                  uint16_t* __restrict__ h_out, bool q_tiled) {
  __shared__ float red[4][32][R];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, lg = lane >> 5;
  const int m = blockIdx.x * 32 + (lane & 31);
  const bool live = m < T;
  const int mc = live ? m : T - 1;
  const uint16_t* gurow = gu + (int64_t)mc * 2 * N;
  v8bf xg[R / 16], xu[R / 16];
#pragma unroll
  for (int h = 0; h < R / 16; ++h) {
    xg[h] = load_bf8(xs + (int64_t)mc * 2 * R + h * 16 + lg * 8);
    xu[h] = load_bf8(xs + (int64_t)mc * 2 * R + R + h * 16 + lg * 8);
  }
  v16f acc = v16f{};  // xS_down partial D[ρ][m]
  const int t0 = blockIdx.y * tiles_per_group;
  for (int t = t0 + w; t < t0 + tiles_per_group; t += 4) {
    const int jb = t * 32;
    float gv[16], uv[16];
    load_tile(gurow, jb, lane, live, gv);
    load_tile(gurow + N, jb, lane, live, uv);
    const v16f lgd = lora_tile<R>(bg + (int64_t)(jb + (lane & 31)) * R + lg * 8, xg);
    const v16f lud = lora_tile<R>(bu + (int64_t)(jb + (lane & 31)) * R + lg * 8, xu);
    float hv[16];
    uint32_t hw[8];  // h as packed bf16 pairs (columns i, i+1)
#pragma unroll
    for (int i = 0; i < 16; i += 2) {
      float g0 = gv[i] + s_g * lgd[i], g1 = gv[i + 1] + s_g * lgd[i + 1];
      float u0 = uv[i] + s_u * lud[i], u1 = uv[i + 1] + s_u * lud[i + 1];
      rnd2(g0, g1);
      rnd2(u0, u1);
      hv[i] = (g0 * fast_sigmoid(g0)) * u0;
      hv[i + 1] = (g1 * fast_sigmoid(g1)) * u1;
      hw[i / 2] = rnd2(hv[i], hv[i + 1]);
    }
    if (kWriteQ) quant_tile(hw, lane, m, live, q, mc, N, q_tiled, jb, s, N / 128);
    if (h_out && live) {
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *reinterpret_cast<uint2*>(h_out + (int64_t)m * N + jb + g * 8 + lg * 4) = make_uint2(hw[2 * g], hw[2 * g + 1]);
    }
    // xS_down: D[ρ][m] += Σ_j ad[ρ, j] h[m, j]; A operand rows ρ = lane % 32 (zero past r)
    const int rho = lane & 31;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      v8bf af = rho < R ? load_bf8_perm(ad + (int64_t)rho * N, jb + 16 * ks, lg) : v8bf{};
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, words_bf8(hw + 4 * ks), acc, 0, 0, 0);
    }
  }
  // acc lane l: m = l % 32, ρ = (i/4)*8 + (l/32)*4 + i%4
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int rho = tile_col(i, lane);
    if (rho < R) red[w][lane & 31][rho] = acc[i];
  }
  __syncthreads();
  for (int idx = threadIdx.x; idx < 32 * R; idx += 256) {
    const int mm = idx / R, rr = idx % R;
    const int row = blockIdx.x * 32 + mm;
    if (row < T)
      part[((int64_t)blockIdx.y * T + row) * R + rr] = ((red[0][mm][rr] + red[1][mm][rr]) + red[2][mm][rr]) + red[3][mm][rr];
  }
}

// --------------------------------------------------------------------------------------------- backward
// Program (blockIdx.x = super-block of SB rows, blockIdx.y = column group of CG columns); 8 waves, each owning
// one 32-column tile of the current 256-column octet.  Outer loop over octets, inner over 32-row blocks.
//   dB_g, dB_u, dA_d: per-wave accumulators over the inner loop (tile transposed through LDS), written to
//     the super-block's partial after it;
//   dxa_g, dxa_u, xS_down: per (row block, octet), the 8 waves' products are summed in LDS (fixed order)
//     and read-modify-written into the column group's [T, 3r] partial (first octet stores).
template <int R, bool kQuant>
__global__ __launch_bounds__(512) void bwd_kernel(
    const uint16_t* __restrict__ gu, const uint16_t* __restrict__ xs, const uint16_t* __restrict__ xsT,
    const uint16_t* __restrict__ dhm, const uint16_t* __restrict__ dxd, const uint16_t* __restrict__ dxdT,
    const uint16_t* __restrict__ bg, const uint16_t* __restrict__ bu, const uint16_t* __restrict__ bgT,
    const uint16_t* __restrict__ buT, const uint16_t* __restrict__ ad, const uint16_t* __restrict__ adT, int T,
    int Tpad, int N, int SB, int CG, float s_g, float s_u, uint8_t* __restrict__ q, uint8_t* __restrict__ s,
    float* __restrict__ dxa_part, float* __restrict__ dbg_part, float* __restrict__ dbu_part,
    float* __restrict__ dad_part, uint16_t* __restrict__ dgu_out, bool q_tiled) {
  __shared__ float red[8][32][3 * R];                               // per-wave dxa | dxa_u | xS products
  __shared__ __attribute__((aligned(16))) uint16_t tr[8][3][32][40];  // per-wave transposed dg, du, h [j][m]
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, lg = lane >> 5;
  const int r0 = blockIdx.x * SB, r1 = min(r0 + SB, Tpad);
  const int c0 = blockIdx.y * CG;
  const int rho = lane & 31;
  for (int oc = 0; oc < CG / 256; ++oc) {
    const int jb = c0 + oc * 256 + w * 32;  // this wave's tile
    const uint16_t* bgrow = bg + (int64_t)(jb + (lane & 31)) * R + lg * 8;
    const uint16_t* burow = bu + (int64_t)(jb + (lane & 31)) * R + lg * 8;
    const uint16_t* adtrow = adT + (int64_t)(jb + (lane & 31)) * R + lg * 8;
    // dB_g, dB_u, dA_d of this tile as D[j][ρ] on the 16x16x32 bf16 MFMA (A = transposed tile rows j, k = m;
    // B = xsᵀ / dxdᵀ rows ρ): lane l holds ρ = l % 16 (+16 h) and j = jb + 16 jh + (l / 16) * 4 + i
    v4f dbg[2][R / 16], dbu[2][R / 16], dad[2][R / 16];
#pragma unroll
    for (int jh = 0; jh < 2; ++jh)
#pragma unroll
      for (int h = 0; h < R / 16; ++h) dbg[jh][h] = dbu[jh][h] = dad[jh][h] = v4f{};
    for (int rb = r0; rb < r1; rb += 32) {
      const int m = rb + (lane & 31);
      const bool live = m < T;
      const int mc = live ? m : T - 1;
      v8bf xg[R / 16], xu[R / 16], xd[R / 16];
#pragma unroll
      for (int h = 0; h < R / 16; ++h) {
        xg[h] = load_bf8(xs + (int64_t)mc * 2 * R + h * 16 + lg * 8);
        xu[h] = load_bf8(xs + (int64_t)mc * 2 * R + R + h * 16 + lg * 8);
        xd[h] = load_bf8(dxd + (int64_t)mc * R + h * 16 + lg * 8);
      }
      float gv[16], uv[16], dv[16];
      load_tile(gu + (int64_t)mc * 2 * N, jb, lane, live, gv);
      load_tile(gu + (int64_t)mc * 2 * N + N, jb, lane, live, uv);
      load_tile(dhm + (int64_t)mc * N, jb, lane, live, dv);
      const v16f lgd = lora_tile<R>(bgrow, xg);
      const v16f lud = lora_tile<R>(burow, xu);
      const v16f ldd = lora_tile<R>(adtrow, xd);
      float dgv[16], duv[16], hv[16];
      uint32_t dgw[8], duw[8], hw[8];  // the same as packed bf16 pairs
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        float g0 = gv[i] + s_g * lgd[i], g1 = gv[i + 1] + s_g * lgd[i + 1];
        float u0 = uv[i] + s_u * lud[i], u1 = uv[i + 1] + s_u * lud[i + 1];
        float d0 = dv[i] + ldd[i], d1 = dv[i + 1] + ldd[i + 1];
        rnd2(g0, g1);
        rnd2(u0, u1);
        rnd2(d0, d1);  // dh
        const float sg0 = fast_sigmoid(g0), sg1 = fast_sigmoid(g1);
        const float sl0 = g0 * sg0, sl1 = g1 * sg1;
        hv[i] = sl0 * u0;
        hv[i + 1] = sl1 * u1;
        hw[i / 2] = rnd2(hv[i], hv[i + 1]);
        duv[i] = d0 * sl0;
        duv[i + 1] = d1 * sl1;
        duw[i / 2] = rnd2(duv[i], duv[i + 1]);
        dgv[i] = ((d0 * u0) * sg0) * (g0 * (1.0f - sg0) + 1.0f);
        dgv[i + 1] = ((d1 * u1) * sg1) * (g1 * (1.0f - sg1) + 1.0f);
        dgw[i / 2] = rnd2(dgv[i], dgv[i + 1]);
      }
      if (!live) {
#pragma unroll
        for (int i = 0; i < 8; ++i) dgw[i] = duw[i] = hw[i] = 0u;
      }
      if (dgu_out && live) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          uint16_t* o = dgu_out + (int64_t)m * 2 * N + jb + g * 8 + lg * 4;
          *reinterpret_cast<uint2*>(o) = make_uint2(dgw[2 * g], dgw[2 * g + 1]);
          *reinterpret_cast<uint2*>(o + N) = make_uint2(duw[2 * g], duw[2 * g + 1]);
        }
      }
      if (kQuant) {
        quant_tile(dgw, lane, m, live, q, mc, 2 * N, q_tiled, jb, s, 2 * N / 128);
        quant_tile(duw, lane, m, live, q, mc, 2 * N, q_tiled, N + jb, s, 2 * N / 128);
      }
      // dxa_g | dxa_u | xS_down products over this tile's 32 columns: D[ρ][m]
      v16f pg = v16f{}, pu = v16f{}, px = v16f{};
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const bool ok = rho < R;
        const v8bf fg = ok ? load_bf8_perm(bgT + (int64_t)rho * N, jb + 16 * ks, lg) : v8bf{};
        const v8bf fu = ok ? load_bf8_perm(buT + (int64_t)rho * N, jb + 16 * ks, lg) : v8bf{};
        const v8bf fa = ok ? load_bf8_perm(ad + (int64_t)rho * N, jb + 16 * ks, lg) : v8bf{};
        pg = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fg, words_bf8(dgw + 4 * ks), pg, 0, 0, 0);
        pu = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fu, words_bf8(duw + 4 * ks), pu, 0, 0, 0);
        px = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa, words_bf8(hw + 4 * ks), px, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int rr = tile_col(i, lane);
        if (rr < R) {
          red[w][lane & 31][rr] = pg[i];
          red[w][lane & 31][R + rr] = pu[i];
          red[w][lane & 31][2 * R + rr] = px[i];
        }
      }
      // transpose dg, du, h to [j][m] for the products that reduce over m
#pragma unroll
      for (int i = 0; i < 16; i += 2) {
        const int j = tile_col(i, lane);
        tr[w][0][j][lane & 31] = (uint16_t)dgw[i / 2];
        tr[w][0][j + 1][lane & 31] = (uint16_t)(dgw[i / 2] >> 16);
        tr[w][1][j][lane & 31] = (uint16_t)duw[i / 2];
        tr[w][1][j + 1][lane & 31] = (uint16_t)(duw[i / 2] >> 16);
        tr[w][2][j][lane & 31] = (uint16_t)hw[i / 2];
        tr[w][2][j + 1][lane & 31] = (uint16_t)(hw[i / 2] >> 16);
      }
      __syncthreads();
      // D[j][ρ] += Σ_m dg[m, j] xs_g[m, ρ] etc. over the 32 rows of this block (one K = 32 step)
      {
        const int mo = (lane >> 4) * 8;  // this lane's 8 rows of the block
#pragma unroll
        for (int h = 0; h < R / 16; ++h) {
          const int rr = h * 16 + (lane & 15);
          const v8bf bgx = load_bf8(xsT + (int64_t)rr * Tpad + rb + mo);
          const v8bf bux = load_bf8(xsT + (int64_t)(R + rr) * Tpad + rb + mo);
          const v8bf bdx = load_bf8(dxdT + (int64_t)rr * Tpad + rb + mo);
#pragma unroll
          for (int jh = 0; jh < 2; ++jh) {
            const int jl = jh * 16 + (lane & 15);
            dbg[jh][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(load_bf8(&tr[w][0][jl][mo]), bgx, dbg[jh][h], 0, 0, 0);
            dbu[jh][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(load_bf8(&tr[w][1][jl][mo]), bux, dbu[jh][h], 0, 0, 0);
            dad[jh][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(load_bf8(&tr[w][2][jl][mo]), bdx, dad[jh][h], 0, 0, 0);
          }
        }
      }
      // sum the 8 waves' dxa | xS products and accumulate into the column group's partial
      for (int idx = threadIdx.x; idx < 32 * 3 * R; idx += 512) {
        const int mm = idx / (3 * R), cc = idx % (3 * R);
        const int row = rb + mm;
        if (row < T) {
          float v = red[0][mm][cc];
#pragma unroll
          for (int k = 1; k < 8; ++k) v += red[k][mm][cc];
          float* dst = dxa_part + ((int64_t)blockIdx.y * T + row) * 3 * R + cc;
          *dst = oc == 0 ? v : *dst + v;
        }
      }
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

// out[i] = cast(scale * Σ_p part[p * count + i]), p ascending
template <bool kBf16>
__global__ __launch_bounds__(256) void sum_parts_kernel(const float* __restrict__ part, int64_t n_parts,
                                                        int64_t count, float scale, void* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= count) return;
  float v = part[i];
  for (int64_t p = 1; p < n_parts; ++p) v += part[p * count + i];
  v *= scale;
  if (kBf16) reinterpret_cast<uint16_t*>(out)[i] = (uint16_t)f32_to_bf16_bits(v);
  else reinterpret_cast<float*>(out)[i] = v;
}

}  // namespace

extern "C" int mxfp8_mlp_fwd(const void* gu, const void* xs, const void* bg, const void* bu, const void* ad, int64_t T,
                             int64_t N, int64_t r, float s_g, float s_u, void* q_h, void* s_h, float* part,
                             int64_t n_groups, void* h_out, int64_t q_layout, void* stream) {
  MX_CHECK_ARG(gu && xs && bg && bu && ad && part, "mxfp8_mlp_fwd: null pointer");
  MX_CHECK_ARG(q_layout == 0 || q_layout == 1, "mxfp8_mlp_fwd: q_layout must be 0 (row-major) or 1 (MX-tiled)");
  MX_CHECK_ARG((q_h == nullptr) == (s_h == nullptr), "mxfp8_mlp_fwd: q_h and s_h go together");
  MX_CHECK_ARG(T > 0 && N > 0 && N % 128 == 0 && (r == 16 || r == 32), "mxfp8_mlp_fwd: bad shape");
  MX_CHECK_ARG(T * 2 * N < (1LL << 31), "mxfp8_mlp_fwd: T * 2N must stay below 2^31");
  MX_CHECK_ARG(n_groups > 0 && (N / 32) % n_groups == 0, "mxfp8_mlp_fwd: n_groups must divide N / 32");
  MX_CHECK_ARG(mx_aligned(gu, 16) && mx_aligned(xs, 16) && mx_aligned(bg, 16) && mx_aligned(bu, 16) &&
                   mx_aligned(ad, 16) && mx_aligned(part, 16) && (!q_h || mx_aligned(q_h, 16)) &&
                   (!h_out || mx_aligned(h_out, 16)),
               "mxfp8_mlp_fwd: misaligned buffer");
  const int64_t Tpad = (T + 127) / 128 * 128;
  dim3 grid((unsigned)(Tpad / 32), (unsigned)n_groups);
  const int tpg = (int)(N / 32 / n_groups);
  hipStream_t stm = (hipStream_t)stream;
#define FWD_ARGS (const uint16_t*)gu, (const uint16_t*)xs, (const uint16_t*)bg, (const uint16_t*)bu, (const uint16_t*)ad, \
                 (int)T, (int)N, tpg, s_g, s_u, (uint8_t*)q_h, (uint8_t*)s_h, part, (uint16_t*)h_out, q_layout == 1
  if (r == 16) {
    if (q_h) fwd_kernel<16, true><<<grid, 256, 0, stm>>>(FWD_ARGS);
    else fwd_kernel<16, false><<<grid, 256, 0, stm>>>(FWD_ARGS);
  } else {
    if (q_h) fwd_kernel<32, true><<<grid, 256, 0, stm>>>(FWD_ARGS);
    else fwd_kernel<32, false><<<grid, 256, 0, stm>>>(FWD_ARGS);
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
  MX_CHECK_ARG(q_layout == 0 || q_layout == 1, "mxfp8_mlp_bwd: q_layout must be 0 (row-major) or 1 (MX-tiled)");
  MX_CHECK_ARG(gu && xs && xsT && dhm && dxd && dxdT && bg && bu && bgT && buT && ad && adT && dxa_part &&
                   dbg_part && dbu_part && dad_part,
               "mxfp8_mlp_bwd: null pointer");
  MX_CHECK_ARG((q == nullptr) == (s == nullptr), "mxfp8_mlp_bwd: q and s go together");
  MX_CHECK_ARG(T > 0 && N > 0 && N % 256 == 0 && (r == 16 || r == 32), "mxfp8_mlp_bwd: bad shape (N %% 256)");
  MX_CHECK_ARG(T * 2 * N < (1LL << 31), "mxfp8_mlp_bwd: T * 2N must stay below 2^31");
  MX_CHECK_ARG(SB > 0 && SB % 128 == 0 && CG > 0 && CG % 256 == 0 && N % CG == 0,
               "mxfp8_mlp_bwd: SB must be a multiple of 128, CG a multiple of 256 dividing N");
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
                 q_layout == 1
  if (r == 16) {
    if (q) bwd_kernel<16, true><<<grid, 512, 0, stm>>>(BWD_ARGS);
    else bwd_kernel<16, false><<<grid, 512, 0, stm>>>(BWD_ARGS);
  } else {
    if (q) bwd_kernel<32, true><<<grid, 512, 0, stm>>>(BWD_ARGS);
    else bwd_kernel<32, false><<<grid, 512, 0, stm>>>(BWD_ARGS);
  }
#undef BWD_ARGS
  MX_CHECK_LAUNCH("mxfp8_mlp_bwd");
  return MXFP8_OK;
}

extern "C" int mxfp8_sum_parts(const float* part, int64_t n_parts, int64_t count, float scale, void* out,
                               int out_bf16, void* stream) {
  MX_CHECK_ARG(part && out && n_parts > 0 && count >= 0, "mxfp8_sum_parts: bad arguments");
  if (count == 0) return MXFP8_OK;
  const int64_t blocks = (count + 255) / 256;
  MX_CHECK_ARG(blocks < (1LL << 31), "mxfp8_sum_parts: too large");
  hipStream_t stm = (hipStream_t)stream;
  if (out_bf16) sum_parts_kernel<true><<<(unsigned)blocks, 256, 0, stm>>>(part, n_parts, count, scale, out);
  else sum_parts_kernel<false><<<(unsigned)blocks, 256, 0, stm>>>(part, n_parts, count, scale, out);
  MX_CHECK_LAUNCH("mxfp8_sum_parts");
  return MXFP8_OK;
}
