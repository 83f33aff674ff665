// Device helpers shared by the MXFP8 kernels (gfx950 only).
//
// Numeric contract (reference: /root/reference/scripts/mxfp8.py:46-75, fused_mlp.py:40-62):
//   amax  = max |v| over a 32-element block, NaN if any element is NaN
//   e     = E8M0 round-up of amax / 448 (satfinite): 255 for NaN, 254 for inf, 0 for amax <= 448 * 2^-127
//   code  = RNE E4M3FN of clamp(v * 2^(127 - e), -448, 448)   (e == 0 scales by 1, e == 255 -> code 0x7F)
// The exponent uses the division-free closed form on the amax bit pattern: with amax = (1 + m/2^23) 2^(E-127)
// and 448 = 1.75 * 2^8, ceil(log2(amax / 448)) = E - 135 + [m > 0x600000]; the fp32 quotient of the reference
// never rounds across a power of two, so both routes agree for every fp32 amax.
//
// Register layouts of the gfx950 matrix instructions used here (measured on the device):
//   v_mfma_scale_f32_32x32x64_f8f6f4 (e4m3 x e4m3): operand lane l, byte j holds row l%32 and
//     k = 32*(j/16) + 16*(l/32) + j%16; the E8M0 scale of (row r, 32-block kb) is read from lane r + 32*kb,
//     byte op_sel of the 32-bit scale register.
//   v_mfma_f32_32x32x16_bf16: operand lane l, element i holds row l%32, k = 8*(l/32) + i.
//   32x32 f32 accumulators: lane l, register i holds row (i/4)*8 + (l/32)*4 + i%4, column l%32.
//   v_cvt_pk_fp8_f32 converts to OCP E4M3FN with round-to-nearest-even (bit-exact with an RNE reference for
//     every bf16 input in [-448, 448]); NaN converts to 0x7F / 0xFF.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mxk {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// fp32 -> bf16 bits, round to nearest even; NaN stays a (quiet) NaN.
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) | 0x40u) & 0xffffu;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ float round_bf16(float f) { return __uint_as_float(f32_to_bf16_bits(f) << 16); }
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return f32_to_bf16_bits(lo) | (f32_to_bf16_bits(hi) << 16);
}

// |v| bit pattern: for non-negative floats the unsigned order is the float order and every NaN pattern is
// above +inf, so an unsigned max over these propagates NaN (tl.maximum(..., propagate_nan=ALL)).
__device__ __forceinline__ uint32_t abs_bits(float v) { return __float_as_uint(v) & 0x7fffffffu; }

// E8M0 exponent from the amax bit pattern (sign already cleared).
__device__ __forceinline__ uint32_t e8m0_from_amax_bits(uint32_t b) {
  uint32_t E = b >> 23, m = b & 0x7fffffu;
  int e = (int)E - 8 + (m > 0x600000u ? 1 : 0);
  e = e < 0 ? 0 : e;
  if (E == 255u) e = m ? 255 : 254;
  return (uint32_t)e;
}

// Exponent shift applied to the elements of a block with scale byte e (e != 255).
__device__ __forceinline__ int e8m0_shift(uint32_t e) { return e == 0u ? 0 : 127 - (int)e; }

__device__ __forceinline__ float scale_clamp(float v, int sh) {
  float t = __builtin_ldexpf(v, sh);
  return __builtin_fminf(__builtin_fmaxf(t, -448.0f), 448.0f);
}

// Four block elements -> four E4M3 codes packed little-endian in one dword.
__device__ __forceinline__ uint32_t encode4(float a, float b, float c, float d, uint32_t e) {
  if (e == 255u) return 0x7f7f7f7fu;
  int sh = e8m0_shift(e);
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(scale_clamp(a, sh), scale_clamp(b, sh), 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(scale_clamp(c, sh), scale_clamp(d, sh), w, true);
  return (uint32_t)w;
}

// Byte offset of the scale of (row i, 32-block b) in the 128x4 blocked layout with n_col_tiles tiles of
// 128 columns per row of tiles.
__device__ __forceinline__ int64_t blocked_offset(int64_t i, int64_t b, int64_t n_col_tiles) {
  return ((i >> 7) * n_col_tiles + (b >> 2)) * 512 + (i & 31) * 16 + ((i & 127) >> 5) * 4 + (b & 3);
}

// Byte offset of code (row r, column k) in the MX-tiled layout of an operand with K codes per row: blocks of
// 16 rows x 64 codes stored as contiguous 1 KB, block (r/16, k/64) at ((r/16) * (K/64) + k/64) * 1024; inside
// a block row r%16 takes 64 bytes whose 16-byte chunk c (codes 16c..16c+15 of the block) sits at position
// c ^ ((r >> 2) & 3).  This is byte for byte the image the GEMM keeps in LDS for one 16-row slice of a K step
// (the swizzle spreads a ds_read_b128 over the 64 banks), so one global_load_lds_dwordx4 moves a whole block.
__device__ __forceinline__ int64_t tiled_offset(int64_t r, int64_t k, int64_t K) {
  return ((r >> 4) * (K >> 6) + (k >> 6)) * 1024 + (r & 15) * 64 + ((((k >> 4) & 3) ^ ((r >> 2) & 3)) << 4) +
         (k & 15);
}

// Element offset of (row r, column c) in the fused-tile (FT) layout of a bf16 [R, C] matrix (C % 32 == 0, rows
// padded to a multiple of 32): 32 x 32 blocks of 2 KB, block (r/32, c/32) at ((r/32) * (C/32) + c/32) * 1024
// elements.  Inside a block, columns c%32 = 16 lg + i of row r%32 belong to lane l = r%32 + 32 lg of the fused
// kernels' tile order (a lane's 16 contiguous columns); the block holds first every lane's columns i = 0..7
// (16 bytes per lane, in lane order), then every lane's i = 8..15.  So a wave's two 16-byte loads of a tile
// read two contiguous 1 KB pieces (8 full cache lines each, against 32 half-used lines for a row-major
// matrix), and 4 consecutive columns (c % 4 == 0) are 8 contiguous bytes, the GEMM epilogue's store unit.
__device__ __forceinline__ int64_t ft_offset(int64_t r, int64_t c, int64_t C) {
  return ((r >> 5) * (C >> 5) + (c >> 5)) * 1024 + ((c >> 3) & 1) * 512 + ((r & 31) + 32 * ((c >> 4) & 1)) * 8 +
         (c & 7);
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Running max of the bf16 magnitudes of a packed pair (v_pk_max_u16): for bf16 bit patterns with the sign
// cleared, unsigned 16-bit order is magnitude order and every NaN sorts above +inf, so the max propagates NaN.
__device__ __forceinline__ u16x2 absmax2(u16x2 acc, uint32_t w) {
  return __builtin_elementwise_max(acc, __builtin_bit_cast(u16x2, w & 0x7fff7fffu));
}
// fp32 bit pattern of the larger half (the block amax as fp32 bits)
__device__ __forceinline__ uint32_t amax_bits(u16x2 m) { return (uint32_t)max(m.x, m.y) << 16; }

// Four bf16 (two packed words) of a block with scale byte e -> four E4M3 codes.  Finite blocks (e <= 253)
// use v_cvt_scalef32_pk_fp8_bf16, which computes RNE_E4M3(x / scale) (verified bit-exact on the device for
// every finite bf16 input and power-of-two scale); x / 2^(e-127) = x * 2^(127-e) exactly, and e == 0 scales
// by 1.  RCEIL guarantees |x| / scale <= 448 there, so no clamp is needed.  Blocks with NaN (e = 255) or inf
// (e = 254) take encode4, which clamps inf to +-448 and writes 0x7F for NaN blocks; the choice is made per
// wave (ballot) so the common path stays branch- and select-free.
__device__ __forceinline__ uint32_t encode4_bf16(uint32_t w0, uint32_t w1, uint32_t e) {
  const float sc = __uint_as_float(e == 0u ? 0x3f800000u : e << 23);
  s16x2 r = {0, 0};
  r = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(r, __builtin_bit_cast(bf16x2, w0), sc, false);
  r = __builtin_amdgcn_cvt_scalef32_pk_fp8_bf16(r, __builtin_bit_cast(bf16x2, w1), sc, true);
  uint32_t c = __builtin_bit_cast(uint32_t, r);
  if (__builtin_amdgcn_ballot_w64(e >= 254u)) {
    if (e >= 254u) c = encode4(bf16_lo(w0), bf16_hi(w0), bf16_lo(w1), bf16_hi(w1), e);
  }
  return c;
}

// The pair {v[l], v[l ^ 32]} (pair32) or {v[l], v[l ^ 16]} (pair16) in every lane l, in either order, from one
// v_permlane32_swap / v_permlane16_swap of v with itself: it exchanges rows of 16 lanes between its two
// operands in the VALU, where __shfl_xor goes through LDS (ds_bpermute) and a wait on its return.
__device__ __forceinline__ void pair32(uint32_t v, uint32_t& a, uint32_t& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
  a = r[0];
  b = r[1];
}
__device__ __forceinline__ void pair16(uint32_t v, uint32_t& a, uint32_t& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
  a = r[0];
  b = r[1];
}

// Unsigned max over a 4-lane group (the 4 lanes that share one 32-element block), by DPP quad permutations in
// the VALU (lane l ^ 1: quad_perm 1,0,3,2; lane l ^ 2: quad_perm 2,3,0,1).  Every lane of the wave must be active.
__device__ __forceinline__ uint32_t quad_umax(uint32_t v) {
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, true));
  v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, true));
  return v;
}


typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v8bf as_bf8(uint4 u) {
  u32x4 v = {u.x, u.y, u.z, u.w};
  return __builtin_bit_cast(v8bf, v);
}

// 8 bf16 at p (16 bytes) as a matrix-instruction operand
__device__ __forceinline__ v8bf load_bf8(const uint16_t* p) { return as_bf8(*reinterpret_cast<const uint4*>(p)); }

// 16 contiguous bf16 at p (32 bytes) as 8 packed words
__device__ __forceinline__ void load16(const uint16_t* p, uint32_t* w) {
  const uint4 a = *reinterpret_cast<const uint4*>(p), b = *reinterpret_cast<const uint4*>(p + 8);
  w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
}

// 16 bf16 of row r, columns c0..c0+15 (c0 % 16 == 0) of a [*, C] matrix, row-major (row stride C) or FT
__device__ __forceinline__ void load16_rc(const uint16_t* base, int64_t r, int64_t c0, int64_t C, bool ft,
                                          uint32_t* w) {
  const uint16_t* p = base + (ft ? ft_offset(r, c0, C) : r * C + c0);
  const uint4 a = *reinterpret_cast<const uint4*>(p), b = *reinterpret_cast<const uint4*>(p + (ft ? 512 : 8));
  w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
  w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
}

// load16_rc with non-temporal loads (a stream read once: evict-first in the caches)
__device__ __forceinline__ void load16_rc_nt(const uint16_t* base, int64_t r, int64_t c0, int64_t C, bool ft,
                                             uint32_t* w) {
  typedef unsigned int u32x4n __attribute__((ext_vector_type(4)));
  const uint16_t* p = base + (ft ? ft_offset(r, c0, C) : r * C + c0);
  const u32x4n a = __builtin_nontemporal_load(reinterpret_cast<const u32x4n*>(p));
  const u32x4n b = __builtin_nontemporal_load(reinterpret_cast<const u32x4n*>(p + (ft ? 512 : 8)));
  w[0] = a[0]; w[1] = a[1]; w[2] = a[2]; w[3] = a[3];
  w[4] = b[0]; w[5] = b[1]; w[6] = b[2]; w[7] = b[3];
}

// MX-quantize the 16 contiguous values w (8 packed pairs) of row mc, columns k0..k0+15, which with the partner
// lane's 16 form one 32-block: one 16-byte code store (row-major with Kq codes per row, or MX-tiled), scale
// byte of row m (0 for padded rows).
// Stores of MX codes and scale bytes.  Non-temporal (streaming) stores measured much faster for the write-once
// code streams of the standalone quantizer ([10752, 12288]: 5.3 -> 6.6 TB/s).  MX_NT_QUANT selects them for the
// standalone quantizer kernels, MX_NT_FUSED for the codes the fused kernels write (quant16 and its callers).
#ifndef MX_NT_QUANT
#define MX_NT_QUANT 1
#endif
#ifndef MX_NT_FUSED
#define MX_NT_FUSED 0
#endif
typedef unsigned int u32x2v __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4v __attribute__((ext_vector_type(4)));
template <bool kNt>
__device__ __forceinline__ void store_codes(uint8_t* p, uint4 c) {
  if constexpr (kNt) {
    const u32x4v v = {c.x, c.y, c.z, c.w};
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4v*>(p));
  } else {
    *reinterpret_cast<uint4*>(p) = c;
  }
}
template <bool kNt>
__device__ __forceinline__ void store_codes(uint8_t* p, uint2 c) {
  if constexpr (kNt) {
    const u32x2v v = {c.x, c.y};
    __builtin_nontemporal_store(v, reinterpret_cast<u32x2v*>(p));
  } else {
    *reinterpret_cast<uint2*>(p) = c;
  }
}
template <bool kNt>
__device__ __forceinline__ void store_codes(uint8_t* p, uint32_t c) {
  if constexpr (kNt) __builtin_nontemporal_store(c, reinterpret_cast<uint32_t*>(p));
  else *reinterpret_cast<uint32_t*>(p) = c;
}
template <bool kNt>
__device__ __forceinline__ void store_scale(uint8_t* p, uint8_t e) {
  if constexpr (kNt) __builtin_nontemporal_store(e, p);
  else *p = e;
}

// The 16 codes of w (with the partner lane's 16 forming the 32-block) into c; returns the block's E8M0 scale.
__device__ __forceinline__ uint32_t quant16_codes(const uint32_t* w, uint4& c) {
  u16x2 mm = {0, 0};
#pragma unroll
  for (int k = 0; k < 8; ++k) mm = absmax2(mm, w[k]);
  uint32_t a, b;
  pair32(amax_bits(mm), a, b);  // the partner lane l ^ 32 holds the block's other 16 values
  const uint32_t e = e8m0_from_amax_bits(max(a, b));
  c = make_uint4(encode4_bf16(w[0], w[1], e), encode4_bf16(w[2], w[3], e), encode4_bf16(w[4], w[5], e),
                 encode4_bf16(w[6], w[7], e));
  return e;
}

// The stores of quant16: codes c of row mc, scale byte e of row m (0 for padded rows)
__device__ __forceinline__ void quant16_store(uint4 c, uint32_t e, int m, bool live, uint8_t* q, int64_t mc,
                                              int64_t Kq, bool tiled, int64_t k0, uint8_t* s, int64_t s_col_tiles) {
  store_codes<MX_NT_FUSED>(q + (tiled ? tiled_offset(mc, k0, Kq) : mc * Kq + k0), c);
  // both lanes of the pair store the same byte (no divergent branch in the loop)
  store_scale<MX_NT_FUSED>(s + blocked_offset(m, k0 >> 5, s_col_tiles), live ? (uint8_t)e : (uint8_t)0);
}

__device__ __forceinline__ void quant16(const uint32_t* w, int lane, int m, bool live, uint8_t* q, int64_t mc,
                                        int64_t Kq, bool tiled, int64_t k0, uint8_t* s, int64_t s_col_tiles) {
  uint4 c;
  const uint32_t e = quant16_codes(w, c);
  quant16_store(c, e, m, live, q, mc, Kq, tiled, k0, s, s_col_tiles);
}

typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));

// Round a pair to bf16 with v_cvt_pk_bf16_f32 (round to nearest even, verified bit-exact against a software
// RNE on the device); returns the packed pair and leaves the bf16-valued floats in a, b.
__device__ __forceinline__ uint32_t rnd2(float& a, float& b) {
  const v2f f = {a, b};
  const uint32_t w = __builtin_bit_cast(uint32_t, __builtin_convertvector(f, v2bf));
  a = __uint_as_float(w << 16);
  b = __uint_as_float(w & 0xffff0000u);
  return w;
}

// ---- rank-r products in the fused kernels' column order
// The LoRA-B product D[a][m] = Σ_ρ W[j(a), ρ] X[m, ρ] may take any weight row for MFMA row a; with j(a) = pi_col(a)
// lane l holds, for row m = l % 32, the 16 CONTIGUOUS columns (l/32)*16 + i in its 16 accumulator registers i.
__device__ __forceinline__ int pi_col(int a) { return ((a >> 2) & 1) * 16 + (a >> 3) * 4 + (a & 3); }

// D[a][m] = Σ_ρ W[jb + pi_col(a), ρ] · X[m, ρ] from the lane's weight-row fragments wf (lane l holds weight row
// jb + pi_col(l % 32), k = h*16 + (l/32)*8 .. +7 in wf[h])
template <int R>
__device__ __forceinline__ v16f lora_pi(const v8bf* wf, const v8bf* xf) {
  v16f d = v16f{};
#pragma unroll
  for (int h = 0; h < R / 16; ++h) d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[h], xf[h], d, 0, 0, 0);
  return d;
}

// sigmoid(g) = 1 / (1 + exp(-g)) with the hardware exp2 and reciprocal (about 1 ulp each; the reference's
// Triton fp32 division is approximate as well); silu(g) = g * sigmoid(g).  exp(-g) overflowing to +inf
// gives sigmoid 0 and silu -0, as g / (exp(-g) + 1) does.
__device__ __forceinline__ float fast_sigmoid(float g) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(g * -1.4426950408889634f));
}

// ---- LDS DMA (global_load_lds_dwordx4) and explicit memory-counter waits
typedef __attribute__((address_space(3))) void* lds_ptr_t;
__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(lds_ptr_t)p; }

// global_load_lds_dwordx4: lane i's 16 bytes land at LDS address m0 + 16 i.  Issued from inline assembly so
// the compiler does not treat every later LDS read as dependent on every outstanding DMA (it cannot tell ring
// stages apart and would drain a ring with vmcnt(0)); the kernels order them with explicit vmcnt waits and
// barriers.  m0 is written here and nowhere else in this library's kernels.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds), "v"(g) : "memory", "m0");
}
#pragma clang diagnostic pop

// s_waitcnt vmcnt(N) leaving the other counters unconstrained (gfx9 encoding: vmcnt[3:0] at bits 3:0,
// vmcnt[5:4] at bits 15:14, expcnt at 6:4, lgkmcnt at 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier ordering LDS accesses only: waits for this wave's LDS operations (lgkmcnt), not for its
// outstanding global loads, stores or LDS DMAs, which a __syncthreads() fence would drain.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ---- transposes through LDS with ds_read_b64_tr_b16 (gfx950)
typedef short v4s __attribute__((ext_vector_type(4)));
typedef short v8s16 __attribute__((ext_vector_type(8)));
constexpr int kTrLd = 36;  // bf16 row stride of the per-wave transpose tiles (72 bytes: conflict-free reads)

// 4 bf16 of rows r0 + k (k = 0..3) of column c0 + lane % 16 of a [32][kTrLd] tile.  ds_read_b64_tr_b16 gives
// lane i of each 16-lane group E[i/4 + 4k][i % 4], E[s] being the four bf16 at lane s's address (measured on
// gfx950); lane s therefore points at row r0 + s/4, columns c0 + 4 (s % 4) .. + 3.
__device__ __forceinline__ v4s tr4(const uint16_t* tile, int r0, int c0, int lane) {
  const int sl = lane & 15;
  const uint16_t* p = tile + (r0 + (sl >> 2)) * kTrLd + c0 + 4 * (sl & 3);
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)p);
}

// tr4 / tr_operand over a [32][ld] bf16 tile of another row stride (ld % 4 == 0)
__device__ __forceinline__ v4s tr4_ld(const uint16_t* tile, int ld, int r0, int c0, int lane) {
  const int sl = lane & 15;
  const uint16_t* p = tile + (r0 + (sl >> 2)) * ld + c0 + 4 * (sl & 3);
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4s*)p);
}
__device__ __forceinline__ v8bf tr_operand_ld(const uint16_t* tile, int ld, int c0, int lane) {
  const int g8 = (lane >> 4) * 8;
  const v4s lo = tr4_ld(tile, ld, g8, c0, lane), hi = tr4_ld(tile, ld, g8 + 4, c0, lane);
  const v8s16 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(v8bf, v);
}

// 16x16x32 A operand of the transposed tile: lane l holds column c0 + l % 16, rows 8 (l / 16) + 0..7
__device__ __forceinline__ v8bf tr_operand(const uint16_t* tile, int c0, int lane) {
  const int g8 = (lane >> 4) * 8;
  const v4s lo = tr4(tile, g8, c0, lane), hi = tr4(tile, g8 + 4, c0, lane);
  const v8s16 v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(v8bf, v);
}

// the lane's 16 packed values as row l % 32, columns lg*16 .. + 15 of a [32][kTrLd] tile
__device__ __forceinline__ void tr_store(uint16_t* tile, int lane, const uint32_t* w) {
  uint32_t* p = reinterpret_cast<uint32_t*>(tile + (lane & 31) * kTrLd + (lane >> 5) * 16);
#pragma unroll
  for (int k = 0; k < 8; k += 2) *reinterpret_cast<uint2*>(p + k) = make_uint2(w[k], w[k + 1]);
}

}  // namespace mxk
