/*
 * CPU oracle for the MXFP8 block-32 quantizer.  TEST INFRASTRUCTURE ONLY: this file is compiled into
 * oracle/liboracle_mx.so, which only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load,
 * as the checker.  The product path (the HIP library) never links or calls it.
 *
 * Restates, element by element, the reference quantizer:
 *   - /root/reference/scripts/mxfp8.py:46-75  (_quant_kernel: amax with NaN flag, descale = amax / 448,
 *     cvt.rp.satfinite.ue8m0, rcp selection, clamp to +-448, e4m3 cast, blocked scale store, padded rows = 0)
 *   - /root/reference/scripts/fused_mlp.py:40-62 (_mx_store: the same body writing into a column slice of a
 *     wider destination and its blocked scale layout)
 *   - /root/reference/scripts/mxfp8.py:40-43 (quant_ref = torchao to_mx RCEIL + to_blocked; same math)
 *
 * Two independent routes to the E8M0 exponent are kept so tests can pin one against the other:
 *   oracle_e8m0_ieee   : fp32 division by 448 (IEEE, correctly rounded) then exact ceil(log2) via frexp;
 *   oracle_e8m0_closed : integer closed form on the amax bit pattern (no division).
 * The E4M3 encoder is a nearest-value search over the 127 non-negative finite codes with ties to the
 * even code; it shares no code with the GPU encoder (which uses the hardware convert).
 *
 * Documented choices where the reference is implementation-defined:
 *   - NaN block: scale byte 0xFF (cvt of NaN), every code 0x7F (E4M3FN NaN).  The E8M0 NaN scale already
 *     poisons the block on dequantization, so the code bytes carry no value.
 *   - +-inf amax: satfinite gives the largest finite E8M0 (254); rcp = 2^-127; inf elements clamp to +-448.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float f32_from_bits(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint32_t bits_from_f32(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* mxfp8.py:61-63: descale = amax / 448.0 (fp32); e = cvt.rp.satfinite.ue8m0(descale). */
int oracle_e8m0_ieee(float amax) {
  if (isnan(amax)) return 255;
  volatile float d = amax / 448.0f; /* fp32 division, round to nearest even */
  if (isinf(d)) return 254;          /* satfinite: +inf -> largest finite power of two */
  if (d == 0.0f) return 0;           /* ue8m0 has no zero; the smallest code (2^-127) is the round-up of 0 */
  int ex;
  double f = frexp((double)d, &ex); /* d = f * 2^ex, 0.5 <= f < 1, exact */
  int c = (f == 0.5) ? ex - 1 : ex;  /* ceil(log2(d)) */
  int e = c + 127;
  if (e < 0) e = 0;
  if (e > 254) e = 254;
  return e;
}

/* Same exponent from the amax bit pattern only.  amax = (1 + m/2^23) 2^(E-127) and 448 = 1.75 * 2^8, so
 * ceil(log2(amax/448)) = E - 135 + [m > 0.75 * 2^23]; fp32 rounding of the quotient never crosses a power
 * of two (the quotient's distance from 2^k is at least 0.57 ulp when it lies above it). */
int oracle_e8m0_closed(uint32_t amax_bits) {
  uint32_t E = (amax_bits >> 23) & 0xffu, m = amax_bits & 0x7fffffu;
  if (E == 255u) return m ? 255 : 254;
  if (E == 0u) return 0;
  int e = (int)E - 8 + (m > 0x600000u ? 1 : 0);
  return e < 0 ? 0 : e;
}

/* Value of a non-negative finite E4M3FN code (bias 7, 3 mantissa bits, subnormal step 2^-9). */
static double e4m3_value(int code) {
  int E = (code >> 3) & 0xf, M = code & 7;
  if (E == 0) return ldexp((double)M, -9);
  return ldexp((double)(8 + M), E - 10);
}

static double g_vals[127];
static int g_vals_ready = 0;

static void init_vals(void) {
  if (g_vals_ready) return;
  for (int c = 0; c < 127; ++c) g_vals[c] = e4m3_value(c);
  g_vals_ready = 1;
}

/* Round-to-nearest-even cast of an fp32 value already clamped to [-448, 448] (mxfp8.py:66-67). */
uint8_t oracle_e4m3_rne(float x) {
  init_vals();
  if (isnan(x)) return 0x7f;
  uint8_t sign = signbit(x) ? 0x80 : 0x00;
  double a = fabs((double)x);
  if (a >= 448.0) return sign | 0x7e;
  int lo = 0, hi = 126; /* largest code with value <= a */
  while (lo < hi) {
    int mid = (lo + hi + 1) / 2;
    if (g_vals[mid] <= a) lo = mid; else hi = mid - 1;
  }
  if (g_vals[lo] == a) return sign | (uint8_t)lo;
  double dl = a - g_vals[lo], dh = g_vals[lo + 1] - a;
  int c = dl < dh ? lo : (dh < dl ? lo + 1 : ((lo & 1) ? lo + 1 : lo));
  return sign | (uint8_t)c;
}

/* E4M3FN code -> value (fp32), NaN for 0x7f/0xff. */
float oracle_e4m3_decode(uint8_t code) {
  init_vals();
  if ((code & 0x7f) == 0x7f) return f32_from_bits(0x7fc00000u);
  double v = g_vals[code & 0x7f];
  return (float)((code & 0x80) ? -v : v);
}

/* Byte offset of the scale of (row i, 32-block b) in the 128x4 blocked layout whose rows of tiles hold
 * n_col_tiles tiles of 128 columns (mxfp8.py:74, fused_mlp.py:59-61). */
int64_t oracle_blocked_offset(int64_t i, int64_t b, int64_t n_col_tiles) {
  return ((i / 128) * n_col_tiles + b / 4) * 512 + (i % 32) * 16 + ((i % 128) / 32) * 4 + (b % 4);
}

/*
 * Quantize x[rows, cols] (bf16 bit patterns, row stride ld_x elements) along the columns:
 *   codes -> q[i * ld_q + q_col0 + c]
 *   scale -> s[blocked_offset(i, s_tile0 * 4 + b, s_col_tiles)]
 * and zero the scale bytes of the padded rows rows..ceil(rows/128)*128 of the touched tiles.
 * cols must be a multiple of 32.  Returns 0, or -1 on a bad argument.
 */
int oracle_mx_quant(const uint16_t* x, int64_t rows, int64_t cols, int64_t ld_x, uint8_t* q, int64_t ld_q,
                    int64_t q_col0, uint8_t* s, int64_t s_col_tiles, int64_t s_tile0) {
  if (rows < 0 || cols % 32 != 0 || ld_x < cols || ld_q < q_col0 + cols) return -1;
  int64_t nblk = cols / 32;
  for (int64_t i = 0; i < rows; ++i) {
    const uint16_t* xr = x + i * ld_x;
    for (int64_t b = 0; b < nblk; ++b) {
      float v[32];
      float amax = 0.0f;
      int has_nan = 0;
      for (int k = 0; k < 32; ++k) {
        v[k] = f32_from_bits((uint32_t)xr[b * 32 + k] << 16);
        if (isnan(v[k])) has_nan = 1;
        float a = fabsf(v[k]);
        if (a > amax) amax = a;
      }
      if (has_nan) amax = f32_from_bits(0x7fc00000u); /* mxfp8.py:59-60 */
      int e = oracle_e8m0_ieee(amax);
      uint8_t* qr = q + i * ld_q + q_col0 + b * 32;
      if (e == 255) {
        for (int k = 0; k < 32; ++k) qr[k] = 0x7f;
      } else {
        /* mxfp8.py:64-65: rcp = 2^-127 for e == 254, 1.0 for e == 0, else 2^(127 - e); always exact */
        float rcp = (e == 0) ? 1.0f : (e == 254 ? f32_from_bits(0x00400000u) : ldexpf(1.0f, 127 - e));
        for (int k = 0; k < 32; ++k) {
          float t = v[k] * rcp;
          if (t > 448.0f) t = 448.0f;
          if (t < -448.0f) t = -448.0f;
          qr[k] = oracle_e4m3_rne(t);
        }
      }
      s[oracle_blocked_offset(i, s_tile0 * 4 + b, s_col_tiles)] = (uint8_t)e;
    }
  }
  int64_t rpad = ((rows + 127) / 128) * 128;
  for (int64_t i = rows; i < rpad; ++i)
    for (int64_t b = 0; b < nblk; ++b) s[oracle_blocked_offset(i, s_tile0 * 4 + b, s_col_tiles)] = 0;
  return 0;
}

/* Dequantize codes q[rows, cols] (row stride ld_q) with blocked scales s (n_col_tiles per tile row) to fp32. */
int oracle_mx_dequant(const uint8_t* q, int64_t rows, int64_t cols, int64_t ld_q, const uint8_t* s,
                      int64_t n_col_tiles, float* out) {
  if (rows < 0 || cols % 32 != 0) return -1;
  for (int64_t i = 0; i < rows; ++i)
    for (int64_t c = 0; c < cols; ++c) {
      uint8_t e = s[oracle_blocked_offset(i, c / 32, n_col_tiles)];
      float v = oracle_e4m3_decode(q[i * ld_q + c]);
      out[i * cols + c] = (e == 255) ? f32_from_bits(0x7fc00000u) : ldexpf(v, (int)e - 127);
    }
  return 0;
}

/* Exported for tests that exercise the fp32 bit helpers directly. */
uint32_t oracle_f32_bits(float f) { return bits_from_f32(f); }
