// MXFP8 block-32 quantizer kernels for gfx950: along the rows (K axis), along the columns of a frozen weight
// (transposed axis) in the same pass, and dequantization.
//
// Reference behaviour: /root/reference/scripts/mxfp8.py:46-86 (_quant_kernel, mx_quant), :40-43 (quant_ref),
// /root/reference/scripts/fused_mlp.py:40-62 (_mx_store column slices).  Bytes are identical to the
// reference arithmetic described in mx_device.h.
//
// Codes go out row-major or in the MX-tiled layout the GEMM streams (tiled_offset in mx_device.h).
//
// Work decomposition: one 256-thread workgroup per 128 x 128 tile, which is exactly one 512-byte scale tile.
// Wave w owns the tile's rows 32w..32w+31, so each 32-row block of a column lies inside one wave: lane l
// (rg = l / 16, ch = l % 16) loads columns 8ch..8ch+7 (16 bytes) of rows 32w + 8rg + k, k = 0..7 (one load
// instruction reads 4 whole 256-byte row pieces).
//   Row axis: the 4 lanes of a 32-column block reduce their amax with two lane swaps.
//   Column axis: a column's amax is the max over the lane's 8 registers and the 4 lanes l, l^16, l^32, l^48
//   (two lane swaps, bf16 pairs packed), and its codes come from bf16 pairs of two rows packed with v_perm,
//   through the same scaled conversion as the row axis.  Only the codes of the xᵀ tile go through LDS (16 KB),
//   so 6 workgroups fit on a CU (the register budget); they leave as whole 128-byte row pieces.
// The tile's scale bytes are assembled in LDS and leave as one coalesced 512-byte store.
#include "abi_common.h"
#include "mx_device.h"

using namespace mxk;

namespace {

constexpr int kTile = 128;
constexpr int kThreads = 256;
constexpr int kLdC = kTile + 16;  // byte row stride of the LDS tile of transposed codes (16-B aligned)

// Quantize 8 consecutive bf16 (one uint4) whose 4-lane group forms one 32-block; returns the codes and the
// block's scale byte.
__device__ __forceinline__ uint2 quant8(uint4 v, uint32_t& e_out) {
  u16x2 m = {0, 0};
  m = absmax2(m, v.x);
  m = absmax2(m, v.y);
  m = absmax2(m, v.z);
  m = absmax2(m, v.w);
  const uint32_t am = quad_umax(amax_bits(m));
  const uint32_t e = e8m0_from_amax_bits(am);
  e_out = e;
  return make_uint2(encode4_bf16(v.x, v.y, e), encode4_bf16(v.z, v.w, e));
}

// The low (or high) bf16 halves of a and b as one packed pair, a's in the low half.
__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }
__device__ __forceinline__ uint32_t word(const uint4& v, int p) { return p == 0 ? v.x : p == 1 ? v.y : p == 2 ? v.z : v.w; }

// Six waves per SIMD (80 VGPRs) measured 5-6% faster on the dual-axis weight shapes than the unconstrained 89
// VGPRs (five) and than 64 (eight, with a spill), one box, twice each.
template <bool kRows, bool kCols>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(6, 8))) void quant_kernel(
    const uint16_t* __restrict__ x, int64_t rows, int64_t ld_x, uint8_t* __restrict__ q, int64_t ld_q,
    uint8_t* __restrict__ s, int64_t s_col_tiles, int64_t s_tile0, uint8_t* __restrict__ qt,
    uint8_t* __restrict__ st, int64_t tk) {
  __shared__ uint32_t stile[kTile];                  // row-axis scale tile (512 B)
  __shared__ uint32_t sttile[kCols ? kTile : 1];     // transposed-axis scale tile
  __shared__ __attribute__((aligned(16))) uint8_t qtt[kCols ? kTile * kLdC : 16];  // the xᵀ tile's codes
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int rg = lane >> 4, ch = lane & 15;
  const int64_t ct = blockIdx.x;  // column tile
  const int64_t rt = blockIdx.y;  // row tile
  const int64_t col = ct * kTile + ch * 8;
  const int rl0 = 32 * w + 8 * rg;  // the first of this lane's 8 rows within the tile
  // Every load is issued (rows past the end re-read the last row): loads under a bounds branch each made the
  // compiler wait for all eight before the first row's work.  The row axis never uses those rows' values (their
  // codes are not stored, their scale byte is 0); the column axis takes them as zeros, through a mask (a select
  // let the compiler put the load back under a branch).
  uint4 v[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const int64_t r = rt * kTile + rl0 + k;
    const uint4 t = *reinterpret_cast<const uint4*>(x + min(r, rows - 1) * ld_x + col);
    if constexpr (kCols) {
      const uint32_t m = r < rows ? ~0u : 0u;
      v[k] = make_uint4(t.x & m, t.y & m, t.z & m, t.w & m);
    } else {
      v[k] = t;
    }
  }
  if (kRows) {
    // every byte of the scale tile is written (0 for rows past `rows`), so the tile needs no clearing
    uint8_t* sb = reinterpret_cast<uint8_t*>(stile);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int rl = rl0 + k;
      const int64_t r = rt * kTile + rl;
      uint32_t e;
      const uint2 codes = quant8(v[k], e);
      // row-major (row stride ld_q), or the MX-tiled layout with tk codes per row
      if (r < rows) store_codes<MX_NT_QUANT>(q + (tk ? tiled_offset(r, col, tk) : r * ld_q + col), codes);
      if ((ch & 3) == 0) sb[(rl & 31) * 16 + w * 4 + (ch >> 2)] = r < rows ? (uint8_t)e : (uint8_t)0;
    }
  }
  if (kCols) {
    uint8_t* stb = reinterpret_cast<uint8_t*>(sttile);
#pragma unroll
    for (int p = 0; p < 4; ++p) {  // tile columns c = 8ch + 2p (low halves) and c + 1 (high halves)
      u16x2 m = {0, 0};
#pragma unroll
      for (int k = 0; k < 8; ++k) m = absmax2(m, word(v[k], p));
      uint32_t pa, pb;
      pair16(__builtin_bit_cast(uint32_t, m), pa, pb);
      m = __builtin_elementwise_max(__builtin_bit_cast(u16x2, pa), __builtin_bit_cast(u16x2, pb));
      pair32(__builtin_bit_cast(uint32_t, m), pa, pb);
      m = __builtin_elementwise_max(__builtin_bit_cast(u16x2, pa), __builtin_bit_cast(u16x2, pb));
      const uint32_t e0 = e8m0_from_amax_bits((uint32_t)m.x << 16), e1 = e8m0_from_amax_bits((uint32_t)m.y << 16);
      const uint32_t w0 = word(v[0], p), w1 = word(v[1], p), w2 = word(v[2], p), w3 = word(v[3], p);
      const uint32_t w4 = word(v[4], p), w5 = word(v[5], p), w6 = word(v[6], p), w7 = word(v[7], p);
      // codes of xᵀ rows c, c + 1 (tile-local), columns rl0..rl0+7: one 8-byte slot of each LDS row, slot
      // rl0 / 8 = 4w + rg XOR-swizzled by (c / 8) & 14, which spreads a write instruction over all 64 banks
      // and keeps the slot pairs of a 16-byte read-back together
      const uint2 c0 = make_uint2(encode4_bf16(pack_lo(w0, w1), pack_lo(w2, w3), e0),
                                  encode4_bf16(pack_lo(w4, w5), pack_lo(w6, w7), e0));
      const uint2 c1 = make_uint2(encode4_bf16(pack_hi(w0, w1), pack_hi(w2, w3), e1),
                                  encode4_bf16(pack_hi(w4, w5), pack_hi(w6, w7), e1));
      const int c = ch * 8 + 2 * p;
      const int slot = (4 * w + rg) ^ (ch & 14);
      *reinterpret_cast<uint2*>(qtt + c * kLdC + slot * 8) = c0;
      *reinterpret_cast<uint2*>(qtt + (c + 1) * kLdC + slot * 8) = c1;
      if (rg == 0) {
        stb[(c & 31) * 16 + (c >> 5) * 4 + w] = (uint8_t)e0;
        stb[((c + 1) & 31) * 16 + ((c + 1) >> 5) * 4 + w] = (uint8_t)e1;
      }
    }
  }
  __syncthreads();
  if (kCols) {
    // the xᵀ tile leaves as whole 128-byte row pieces: 8 lanes per row, 16 bytes each, 32 rows per pass
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int rr = (tid >> 3) + 32 * j, ch16 = tid & 7;
      const int slot = (2 * ch16) ^ ((rr >> 3) & 14);
      store_codes<MX_NT_QUANT>(qt + (ct * kTile + rr) * rows + rt * kTile + ch16 * 16,
                               *reinterpret_cast<const uint4*>(qtt + rr * kLdC + slot * 8));
    }
  }
  if (kRows && tid < 32)
    store_codes<MX_NT_QUANT>(s + (rt * s_col_tiles + s_tile0 + ct) * 512 + tid * 16,
                             reinterpret_cast<const uint4*>(stile)[tid]);
  if (kCols && tid >= 64 && tid < 96) {
    // tile (row tile ct, column tile rt) of xᵀ's blocked scales, rows/128 tiles per tile row
    const int64_t n_tiles_t = rows / kTile;
    reinterpret_cast<uint4*>(st + (ct * n_tiles_t + rt) * 512)[tid - 64] =
        reinterpret_cast<const uint4*>(sttile)[tid - 64];
  }
}

__global__ __launch_bounds__(kThreads) void dequant_kernel(const uint8_t* __restrict__ q, int64_t rows,
                                                           int64_t cols, int64_t ld_q,
                                                           const uint8_t* __restrict__ s, int64_t s_col_tiles,
                                                           float* __restrict__ out) {
  const int64_t idx = ((int64_t)blockIdx.x * kThreads + threadIdx.x) * 4;
  const int64_t n = rows * cols;
  if (idx >= n) return;
  const int64_t i = idx / cols, c = idx % cols;  // cols % 128 == 0: the 4 elements share row and block
  const uint32_t e = s[blocked_offset(i, c >> 5, s_col_tiles)];
  const uint32_t w = *reinterpret_cast<const uint32_t*>(q + i * ld_q + c);
  float4 o;
  float* po = reinterpret_cast<float*>(&o);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t code = (w >> (8 * k)) & 0xffu;
    const uint32_t E = (code >> 3) & 0xfu, M = code & 7u;
    float v = E == 0 ? __builtin_ldexpf((float)M, -9) : __builtin_ldexpf((float)(8u + M), (int)E - 10);
    v = (code & 0x80u) ? -v : v;
    if ((code & 0x7fu) == 0x7fu || e == 255u) v = __uint_as_float(0x7fc00000u);
    else v = __builtin_ldexpf(v, (int)e - 127);
    po[k] = v;
  }
  *reinterpret_cast<float4*>(out + idx) = o;
}

// Row-major codes [rows, cols] (row stride ld_q) -> the MX-tiled layout (ceil(rows/16)*16 rows; the rows
// past `rows` in the last 16-row block are zero).  One thread per 16-byte chunk of the output.
__global__ __launch_bounds__(kThreads) void tile_codes_kernel(const uint8_t* __restrict__ q, int64_t rows,
                                                              int64_t cols, int64_t ld_q, uint8_t* __restrict__ out,
                                                              int64_t n_chunks) {
  const int64_t o = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (o >= n_chunks) return;
  const int64_t blk = o >> 6, kbs = cols >> 6;
  const int64_t r = (blk / kbs) * 16 + ((o >> 2) & 15), kb = blk % kbs;
  const int c = (int)(o & 3) ^ (int)((r >> 2) & 3);
  uint4 v = make_uint4(0, 0, 0, 0);
  if (r < rows) v = *reinterpret_cast<const uint4*>(q + r * ld_q + kb * 64 + c * 16);
  reinterpret_cast<uint4*>(out)[o] = v;
}

}  // namespace

extern "C" int mxfp8_quant_rows(const void* x, int64_t rows, int64_t cols, int64_t ld_x, void* q, int64_t ld_q,
                                void* s, int64_t s_col_tiles, int64_t s_tile0, void* stream) {
  MX_CHECK_ARG(x && q && s, "mxfp8_quant_rows: null pointer");
  MX_CHECK_ARG(rows >= 0 && cols > 0 && cols % 128 == 0, "mxfp8_quant_rows: need cols %% 128 == 0 (cols=%lld)",
               (long long)cols);
  MX_CHECK_ARG(ld_x >= cols && ld_x % 8 == 0 && ld_q >= cols && ld_q % 16 == 0,
               "mxfp8_quant_rows: bad strides ld_x=%lld ld_q=%lld", (long long)ld_x, (long long)ld_q);
  MX_CHECK_ARG(s_tile0 >= 0 && s_tile0 + cols / 128 <= s_col_tiles, "mxfp8_quant_rows: scale tiles out of range");
  MX_CHECK_ARG(mx_aligned(x, 16) && mx_aligned(q, 16) && mx_aligned(s, 16), "mxfp8_quant_rows: misaligned buffer");
  if (rows == 0) return MXFP8_OK;
  MX_CHECK_ARG((rows + 127) / 128 <= 0x7fffffff, "mxfp8_quant_rows: too many rows");
  dim3 grid((unsigned)(cols / 128), (unsigned)((rows + 127) / 128));
  quant_kernel<true, false><<<grid, kThreads, 0, (hipStream_t)stream>>>(
      (const uint16_t*)x, rows, ld_x, (uint8_t*)q, ld_q, (uint8_t*)s, s_col_tiles, s_tile0, nullptr, nullptr, 0);
  MX_CHECK_LAUNCH("mxfp8_quant_rows");
  return MXFP8_OK;
}

extern "C" int mxfp8_quant_dual(const void* x, int64_t rows, int64_t cols, int64_t ld_x, void* q, void* s, void* qt,
                                void* st, void* stream) {
  MX_CHECK_ARG(x, "mxfp8_quant_dual: null input");
  MX_CHECK_ARG((q == nullptr) == (s == nullptr) && (qt == nullptr) == (st == nullptr) && (q || qt),
               "mxfp8_quant_dual: each axis needs both codes and scales");
  MX_CHECK_ARG(rows > 0 && cols > 0 && rows % 128 == 0 && cols % 128 == 0,
               "mxfp8_quant_dual: need rows, cols %% 128 == 0 (rows=%lld cols=%lld)", (long long)rows,
               (long long)cols);
  MX_CHECK_ARG(ld_x >= cols && ld_x % 8 == 0, "mxfp8_quant_dual: bad ld_x");
  MX_CHECK_ARG(mx_aligned(x, 16) && (!q || (mx_aligned(q, 16) && mx_aligned(s, 16))) &&
                   (!qt || (mx_aligned(qt, 16) && mx_aligned(st, 16))),
               "mxfp8_quant_dual: misaligned buffer");
  dim3 grid((unsigned)(cols / 128), (unsigned)(rows / 128));
  hipStream_t stm = (hipStream_t)stream;
  if (q && qt)
    quant_kernel<true, true><<<grid, kThreads, 0, stm>>>((const uint16_t*)x, rows, ld_x, (uint8_t*)q, cols,
                                                         (uint8_t*)s, cols / 128, 0, (uint8_t*)qt, (uint8_t*)st, 0);
  else if (q)
    quant_kernel<true, false><<<grid, kThreads, 0, stm>>>((const uint16_t*)x, rows, ld_x, (uint8_t*)q, cols,
                                                          (uint8_t*)s, cols / 128, 0, nullptr, nullptr, 0);
  else
    quant_kernel<false, true><<<grid, kThreads, 0, stm>>>((const uint16_t*)x, rows, ld_x, nullptr, 0, nullptr, 0,
                                                          0, (uint8_t*)qt, (uint8_t*)st, 0);
  MX_CHECK_LAUNCH("mxfp8_quant_dual");
  return MXFP8_OK;
}

extern "C" int mxfp8_quant_tiled(const void* x, int64_t rows, int64_t cols, int64_t ld_x, void* q, void* s,
                                 void* stream) {
  MX_CHECK_ARG(x && q && s, "mxfp8_quant_tiled: null pointer");
  MX_CHECK_ARG(rows >= 0 && cols > 0 && cols % 128 == 0, "mxfp8_quant_tiled: need cols %% 128 == 0 (cols=%lld)",
               (long long)cols);
  MX_CHECK_ARG(ld_x >= cols && ld_x % 8 == 0, "mxfp8_quant_tiled: bad ld_x=%lld", (long long)ld_x);
  MX_CHECK_ARG(mx_aligned(x, 16) && mx_aligned(q, 16) && mx_aligned(s, 16), "mxfp8_quant_tiled: misaligned buffer");
  if (rows == 0) return MXFP8_OK;
  MX_CHECK_ARG((rows + 127) / 128 <= 0x7fffffff, "mxfp8_quant_tiled: too many rows");
  dim3 grid((unsigned)(cols / 128), (unsigned)((rows + 127) / 128));
  quant_kernel<true, false><<<grid, kThreads, 0, (hipStream_t)stream>>>(
      (const uint16_t*)x, rows, ld_x, (uint8_t*)q, 0, (uint8_t*)s, cols / 128, 0, nullptr, nullptr, cols);
  MX_CHECK_LAUNCH("mxfp8_quant_tiled");
  return MXFP8_OK;
}

extern "C" int mxfp8_tile_codes(const void* q, int64_t rows, int64_t cols, int64_t ld_q, void* out, void* stream) {
  MX_CHECK_ARG(q && out, "mxfp8_tile_codes: null pointer");
  MX_CHECK_ARG(rows >= 0 && cols > 0 && cols % 64 == 0 && ld_q >= cols && ld_q % 16 == 0,
               "mxfp8_tile_codes: bad shape (rows=%lld cols=%lld ld_q=%lld)", (long long)rows, (long long)cols,
               (long long)ld_q);
  MX_CHECK_ARG(mx_aligned(q, 16) && mx_aligned(out, 16), "mxfp8_tile_codes: misaligned buffer");
  if (rows == 0) return MXFP8_OK;
  const int64_t n_chunks = (rows + 15) / 16 * 16 * cols / 16;
  const int64_t blocks = (n_chunks + kThreads - 1) / kThreads;
  MX_CHECK_ARG(blocks <= 0x7fffffff, "mxfp8_tile_codes: too large");
  tile_codes_kernel<<<(unsigned)blocks, kThreads, 0, (hipStream_t)stream>>>((const uint8_t*)q, rows, cols, ld_q,
                                                                            (uint8_t*)out, n_chunks);
  MX_CHECK_LAUNCH("mxfp8_tile_codes");
  return MXFP8_OK;
}

extern "C" int mxfp8_dequant(const void* q, int64_t rows, int64_t cols, int64_t ld_q, const void* s,
                             int64_t s_col_tiles, float* out, void* stream) {
  MX_CHECK_ARG(q && s && out, "mxfp8_dequant: null pointer");
  MX_CHECK_ARG(rows >= 0 && cols > 0 && cols % 128 == 0 && ld_q >= cols && ld_q % 4 == 0,
               "mxfp8_dequant: bad shape");
  MX_CHECK_ARG(s_col_tiles >= cols / 128, "mxfp8_dequant: bad s_col_tiles");
  MX_CHECK_ARG(mx_aligned(q, 4) && mx_aligned(out, 16), "mxfp8_dequant: misaligned buffer");
  if (rows == 0) return MXFP8_OK;
  const int64_t n4 = rows * cols / 4;
  const int64_t blocks = (n4 + kThreads - 1) / kThreads;
  MX_CHECK_ARG(blocks <= 0x7fffffff, "mxfp8_dequant: too large");
  dequant_kernel<<<(unsigned)blocks, kThreads, 0, (hipStream_t)stream>>>((const uint8_t*)q, rows, cols, ld_q,
                                                                         (const uint8_t*)s, s_col_tiles, out);
  MX_CHECK_LAUNCH("mxfp8_dequant");
  return MXFP8_OK;
}
