/*
 * C-ABI of the MI355X (gfx950) MXFP8 fused SwiGLU-MLP library, libmxfp8_mlp.so.
 *
 * Plain pointers and sizes only.  Every pointer is a device pointer unless stated otherwise; `stream` is a
 * hipStream_t (NULL = the default stream).  All launches are asynchronous on `stream`; nothing here
 * allocates or frees device memory: callers own every buffer, including scratch.
 *
 * Return value: 0 on success, MXFP8_ERR_ARG (< 0) when an argument check fails (nothing was launched), or
 * a positive hipError_t when a launch failed.  mxfp8_last_error() describes the last failure on the
 * calling thread.
 *
 * MX layout shared by every entry point (reference: /root/reference/scripts/mxfp8.py:36-86):
 *   codes   E4M3FN bytes, row-major with a row stride in elements (bytes);
 *   scales  E8M0 bytes, one per 32 consecutive elements of a row, stored in the 128x4 blocked layout:
 *           byte of (row i, block b) at ((i/128)*n_col_tiles + b/4)*512 + (i%32)*16 + ((i%128)/32)*4 + b%4,
 *           where n_col_tiles = the number of 128-column tiles of the (destination) row; rows past the end up
 *           to the next multiple of 128 hold scale 0.
 */
#ifndef MXFP8_MLP_H
#define MXFP8_MLP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MXFP8_MLP_ABI_VERSION 14
#define MXFP8_OK 0
#define MXFP8_ERR_ARG (-1)
/* mxfp8_gemm_nt layout bits */
#define MXFP8_GEMM_A_TILED 1
#define MXFP8_GEMM_B_TILED 2
#define MXFP8_GEMM_WIDE 4
#define MXFP8_GEMM_C_FT 8
#define MXFP8_GEMM_B_PI 16

/* Returns MXFP8_MLP_ABI_VERSION of the built library (the Python loader refuses a mismatch). */
int mxfp8_abi_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* mxfp8_last_error(void);

/*
 * MX-quantize x[rows, cols] (bf16, row stride ld_x) along its rows (blocks of 32 columns).
 * Replaces mx_quant / _quant_kernel (/root/reference/scripts/mxfp8.py:46-86) and, through the column-slice
 * arguments, _mx_store's writes into a wider destination (/root/reference/scripts/fused_mlp.py:40-62):
 *   codes  -> q[i * ld_q + c]            (q already points at the first destination column)
 *   scales -> s, blocked with s_col_tiles tiles per tile row, starting at column tile s_tile0
 * Padded rows rows..ceil(rows/128)*128 of the touched tiles get scale 0.
 * Requires cols % 128 == 0, 16-byte aligned x/q rows (ld_x % 8 == 0, ld_q % 16 == 0).
 */
int mxfp8_quant_rows(const void* x, int64_t rows, int64_t cols, int64_t ld_x, void* q, int64_t ld_q, void* s,
                     int64_t s_col_tiles, int64_t s_tile0, void* stream);

/*
 * One read of x[rows, cols] (bf16, row stride ld_x) producing both MX operands of a frozen weight:
 *   q [rows, cols] + s   : along the rows (blocks of 32 columns), s_col_tiles = cols / 128
 *   qt[cols, rows] + st  : quantization of xᵀ along its rows (blocks of 32 rows of x), st tiles = rows / 128
 * Replaces quant_ref(w) + quant_ref(w.t().contiguous()) (/root/reference/scripts/mxfp8.py:40-43, :477-478,
 * :488-490).  Either pair may be NULL to skip that axis.  Requires rows % 128 == 0 and cols % 128 == 0.
 */
int mxfp8_quant_dual(const void* x, int64_t rows, int64_t cols, int64_t ld_x, void* q, void* s, void* qt,
                     void* st, void* stream);

/*
 * mxfp8_quant_rows for a whole [rows, cols] bf16 tensor with the codes in the MX-tiled layout: blocks of 16 rows
 * x 64 codes stored as contiguous 1 KB, block (r/16, k/64) at ((r/16) * (cols/64) + k/64) * 1024; inside,
 * row r%16 takes 64 bytes whose 16-byte chunk c sits at position c ^ ((r >> 2) & 3).  q holds
 * ceil(rows/16)*16 rows (the padding rows are not written); scales as mxfp8_quant_rows (cols/128 tiles).
 * Same codes and scales as the reference quantizer (/root/reference/scripts/mxfp8.py:46-86), another byte
 * order: the operand layout of mxfp8_gemm_nt (layout bits), no reference counterpart as a layout.
 */
int mxfp8_quant_tiled(const void* x, int64_t rows, int64_t cols, int64_t ld_x, void* q, void* s, void* stream);

/*
 * Row-major codes [rows, cols] (row stride ld_q, cols % 64 == 0) -> the MX-tiled layout above into out
 * (ceil(rows/16)*16 * cols bytes; padding rows zero).  Used for the frozen weights after enable_mxfp8's
 * quantization (/root/reference/scripts/mxfp8.py:472-494); no reference counterpart as a layout.
 */
int mxfp8_tile_codes(const void* q, int64_t rows, int64_t cols, int64_t ld_q, void* out, void* stream);

/*
 * out[rows, cols] (fp32, dense) = E4M3(q) * 2^(e - 127), NaN where the scale byte is 0xFF.
 * No reference counterpart as a function: the reference dequantizes only inside torch._scaled_mm
 * (/root/reference/scripts/fused_mlp.py:279); this exposes the same arithmetic for checks.
 */
int mxfp8_dequant(const void* q, int64_t rows, int64_t cols, int64_t ld_q, const void* s, int64_t s_col_tiles,
                  float* out, void* stream);

/*
 * C[M, N] (bf16, row stride ldc) = bf16( A[M, K] · B[N, K]ᵀ ) with MX block scales on both operands, fp32
 * accumulation, K-contiguous operands (row strides lda, ldb bytes), scales blocked with K/128 tiles per row.
 * Replaces torch._scaled_mm(A, B.t(), sA, sB, out_dtype=bf16) (/root/reference/scripts/fused_mlp.py:279,
 * :283, :309, :329).
 * Optional rank-r epilogue (lora_p != NULL), replacing the addmm_ that follows (fused_mlp.py:284, :331):
 *   C = bf16( bf16(A·Bᵀ) + alpha * P[M, r] · Q[N, r]ᵀ ),  P, Q bf16 with row strides ld_p, ld_q,
 *   r in {16, 32, 48, 64}.
 * Requires K % 128 == 0, N % 128 == 0, lda/ldb % 16 == 0, ldc % 4 == 0.
 * layout bits: MXFP8_GEMM_A_TILED = A codes in the MX-tiled layout (mxfp8_quant_tiled / mxfp8_tile_codes,
 * lda ignored), MXFP8_GEMM_B_TILED = the same for B (results are bit-identical to row-major operands; the
 * tiled layout lets every DMA of the GEMM move a contiguous 1 KB instead of sixteen 64-byte row pieces);
 * MXFP8_GEMM_WIDE = 8-wave 256 x 256 workgroups, one per CU, instead of the default 4-wave 256 x 128, two per
 * CU (same result bits when no tile is split); MXFP8_GEMM_C_FT = C in the fused-tile (FT) layout instead of
 * row-major (ldc ignored; c holds ceil(M/32)*32 rows, rows past M not written).
 * FT layout of a bf16 [R, C] matrix (C % 32 == 0): 32 x 32 blocks of 2 KB, block (r/32, c/32) at
 * ((r/32) * (C/32) + c/32) * 1024 elements; element (r, c) inside it at ((c/8) % 2) * 512 +
 * (r%32 + 32 * ((c/16) % 2)) * 8 + c % 8.  It is the order in which the fused kernels' waves read a 32 x 32 tile
 * (two contiguous 1 KB pieces); no reference counterpart (the reference keeps gu and dhm row-major).
 * MXFP8_GEMM_B_PI = B holds its rows in the pi_col order inside every 32-row block: B row 32b + a is logical
 * row 32b + pi_col(a), pi_col(a) = ((a >> 2) & 1) * 16 + (a >> 3) * 4 + (a & 3) (mxfp8.fused_dgrad_rows); Q of
 * the rank-r epilogue stays in row order.  C is the same matrix; each lane then holds 16 contiguous columns and
 * stores them as two 16-byte pieces instead of four 8-byte ones.
 * workspace (optional, 256-byte aligned, workspace_bytes long; used with MXFP8_GEMM_WIDE only): when it holds
 * at least mxfp8_gemm_workspace_size(M, N, K) bytes, the tiles of a last wave that would leave more than half
 * of the CUs idle are split along K; their fp32 pieces go through the workspace and are added in a fixed order
 * (the result does not depend on scheduling).  Its first 4 KB are arrival counters that must be zero before
 * the first call (allocate it zeroed); every call leaves them zero.  Calls that share a workspace must not run
 * concurrently.  NULL / too small: every tile runs whole (same result bits as with the split only where no
 * tile was split).
 */
int mxfp8_gemm_nt(const void* a, const void* sa, int64_t lda, const void* b, const void* sb, int64_t ldb,
                  int64_t M, int64_t N, int64_t K, void* c, int64_t ldc, const void* lora_p, int64_t ld_p,
                  const void* lora_q, int64_t ld_q, int64_t r, float alpha, int64_t layout, void* workspace,
                  int64_t workspace_bytes, void* stream);

/*
 * mxfp8_gemm_nt with the output columns in n_seg (1..4) separate row-major matrices: columns
 * [seg_col0[k], seg_col0[k+1]) (the last up to N) go to seg_c[k] with row stride seg_ldc[k]; seg_col0[0] = 0 and
 * every boundary a multiple of 128.  seg_col0, seg_c and seg_ldc are host arrays.  The 4-wave shape with row-major
 * C only (layout bits 0-1), no workspace.  Lets the q|k|v projections of a group run as one GEMM over their
 * concatenated weight while each returns its own contiguous output (the reference runs one _scaled_mm per layer,
 * /root/reference/scripts/fused_linear.py:72-76, :106-109).
 * seg_rcol (host array, or NULL for columns [0, r) everywhere): segment k adds the rank-r product over columns
 * [seg_rcol[k], seg_rcol[k] + r) of P and Q (multiples of 8, within ld_p and ld_q).  A group whose Q is
 * block-diagonal, each layer's B at that layer's own columns of P, then runs rank r per tile instead of the
 * whole width, with the same result (the products it skips are zeros).
 */
int mxfp8_gemm_nt_seg(const void* a, const void* sa, int64_t lda, const void* b, const void* sb, int64_t ldb,
                      int64_t M, int64_t N, int64_t K, int64_t n_seg, const int64_t* seg_col0, void* const* seg_c,
                      const int64_t* seg_ldc, const void* lora_p, int64_t ld_p, const void* lora_q, int64_t ld_q,
                      int64_t r, const int64_t* seg_rcol, float alpha, int64_t layout, void* stream);

/*
 * Bytes of workspace mxfp8_gemm_nt uses for this shape with MXFP8_GEMM_WIDE on the current device (0: no
 * split).  No reference counterpart: torch._scaled_mm (fused_mlp.py:279) manages the cuBLAS workspace itself.
 */
int64_t mxfp8_gemm_workspace_size(int64_t M, int64_t N, int64_t K);

/*
 * Fused SwiGLU forward of the MLP after the gate|up MX GEMM (replaces _fwd_kernel / mlp_fwd,
 * /root/reference/scripts/fused_mlp.py:81-109, :198-215):
 *   gu [T, 2N] bf16 (gate | up), xs [T, 2r] bf16 (xa_gate | xa_up), bg, bu [N, r] bf16, ad [r, N] bf16
 *   g = bf16(gu[:, j] + s_g xs_g·bgᵀ), u = bf16(gu[:, N+j] + s_u xs_u·buᵀ), h = bf16(g / (exp(-g) + 1) * u)
 *   q_h [T, N] + s_h (blocked, N/128 tiles per row, padded rows 0)   = MX(h)       (skipped if q_h == NULL)
 *   part [n_groups, T, r] fp32: xS_down partial sums h·adᵀ over the columns of each of n_groups groups
 *   h_out [T, N] bf16 (optional, may be NULL; needs q_h): h itself, for checks
 *   q_layout bit 0: q_h MX-tiled (see mxfp8_quant_tiled; ceil(T/16)*16 rows) instead of row-major;
 *   q_layout bit 1: gu in the FT layout (see mxfp8_gemm_nt) instead of row-major
 * Requires N % 128 == 0, (N / 32) % n_groups == 0, r in {16, 32}, T * 2N < 2^31.
 */
/*
 * The n_groups mxfp8_mlp_fwd runs best with on the current device (from the kernel's occupancy and the CU
 * count), 0 for an unsupported shape.  The reference sizes its grid with a fixed rule (fused_mlp.py:198-210).
 */
int64_t mxfp8_mlp_fwd_groups(int64_t T, int64_t N, int64_t r);

int mxfp8_mlp_fwd(const void* gu, const void* xs, const void* bg, const void* bu, const void* ad, int64_t T,
                  int64_t N, int64_t r, float s_g, float s_u, void* q_h, void* s_h, float* part, int64_t n_groups,
                  void* h_out, int64_t q_layout, void* stream);

/*
 * Fused SwiGLU backward (replaces _bwd_kernel / mlp_bwd, /root/reference/scripts/fused_mlp.py:112-175,
 * :218-259).  Inputs as in the forward plus dhm [T, N] bf16 (MX(dy)·W_down), dxd [T, r] bf16 (s_d·dy·B_d) and
 * the small transposed copies xsT [2r, Tpad], dxdT [r, Tpad] (zero past T; Tpad = ceil(T/128)*128),
 * bgT, buT [r, N], adT [N, r].  Grid: super-blocks of SB rows (SB % 128 == 0) x column groups of CG columns
 * (CG % 128 == 0, N % CG == 0).  Outputs:
 *   q [T, 2N] + s (2N/128 tiles per row): MX(dg) in columns 0..N-1, MX(du) in N..2N-1  (skipped if q == NULL)
 *   dxa_part [N/128, T, 3r] fp32: dxa_g | dxa_u | xS_down partial sums over each 128-column quad (unscaled);
 *     [N/256, T, 3r] over each 256 columns with q_layout bit 2
 *   dbg_part, dbu_part [ceil(Tpad/SB), N, r] fp32 and dad_part [ceil(Tpad/SB), r, N]: per super-block sums of
 *     dgᵀ·xs_g, duᵀ·xs_u and (hᵀ·dxd)ᵀ (unscaled)
 *   dgu_out [T, 2N] bf16 (optional, may be NULL): dg | du themselves, for checks
 *   q_layout bit 0: q MX-tiled with 2N codes per row (see mxfp8_quant_tiled) instead of row-major;
 *   q_layout bit 1: gu and dhm in the FT layout (see mxfp8_gemm_nt) instead of row-major;
 *   q_layout bit 2: 8-wave workgroups, two quads summed in LDS (CG % 256 == 0, dgu_out NULL), one workgroup per CU
 */
int mxfp8_mlp_bwd(const void* gu, const void* xs, const void* xsT, const void* dhm, const void* dxd,
                  const void* dxdT, const void* bg, const void* bu, const void* bgT, const void* buT, const void* ad,
                  const void* adT, int64_t T, int64_t N, int64_t r, float s_g, float s_u, int64_t SB, int64_t CG,
                  void* q, void* s, float* dxa_part, float* dbg_part, float* dbu_part, float* dad_part,
                  void* dgu_out, int64_t q_layout, void* stream);

/*
 * out[i] = scale * Σ_{p=0..n_parts-1} part[p * count + i], summed in ascending p (deterministic), stored as
 * fp32 or, if out_bf16, rounded to bf16 (RNE).  Replaces the partial-sum reductions part.sum(0) of
 * /root/reference/scripts/fused_mlp.py:214, :258.
 */
int mxfp8_sum_parts(const float* part, int64_t n_parts, int64_t count, float scale, void* out, int out_bf16,
                    void* stream);

/*
 * Per-step bf16 forms of the fp32 LoRA weights (replaces the _cast copies of /root/reference/scripts/
 * fused_mlp.py:272-276 and the transposed copies its kernels index): A_g, A_u [r, K], B_g, B_u [N, r],
 * A_d [r, N], B_d [K, r] -> S = [A_g; A_u] [2r, K], Sᵀ [K, 2r], b_g, b_u [N, r], b_gᵀ, b_uᵀ [r, N], a_d [r, N],
 * a_dᵀ [N, r], b_d [K, r], b_dᵀ [r, K]; round to nearest even.  r <= 64.
 */
int mxfp8_lora_prep(const float* Ag, const float* Au, const float* Bg, const float* Bu, const float* Ad, const float* Bd,
                    int64_t r, int64_t K, int64_t N, void* S, void* ST, void* bg, void* bu, void* bgT, void* buT,
                    void* ad, void* adT, void* bd, void* bdT, void* stream);

/*
 * out[t, ρ] = bf16(x[t, :] · w[ρ, :]), then bf16(out · scale) when scale != 1; x [T, K] bf16 (row stride ld_x),
 * w [rp, K] bf16, out [T, rp] bf16; outT (optional) [rp, Tpad] bf16, the same values transposed and zero for
 * t >= T.  Replaces xs = x2 @ S.t() and dxd = (dy2 @ bd).mul_(s_d) (/root/reference/scripts/fused_mlp.py:277,
 * :311-313).  K % 64 == 0, rp in {16, 32, 64}.
 */
int mxfp8_lora_nt(const void* x, int64_t T, int64_t K, int64_t ld_x, const void* w, int64_t rp, float scale, void* out,
                  void* outT, int64_t Tpad, void* stream);

/*
 * One pass over x [T, K] bf16 (row stride ld_x) giving both mxfp8_quant_tiled(x) (codes q in the MX-tiled
 * layout, ceil(T/16)*16 rows; scales s blocked with K/128 tiles per row, padded rows 0) and
 * mxfp8_lora_nt(x, w, rp, scale, out, outT, Tpad) (out [T, rp] bf16, outT [rp, Tpad] or NULL).  Replaces
 * mx_quant(x2) followed by xs = x2 @ S.t() (/root/reference/scripts/fused_mlp.py:277-279), and mx_quant(dy2)
 * with dxd = (dy2 @ bd).mul_(s_d) (:309-313), each reading the activation once.  K % 128 == 0, rp in {16, 32, 64},
 * Tpad = ceil(T/128)*128.
 */
int mxfp8_quant_lora(const void* x, int64_t T, int64_t K, int64_t ld_x, void* q, void* s, const void* w, int64_t rp,
                     float scale, void* out, void* outT, int64_t Tpad, void* stream);

/*
 * mxfp8_quant_lora plus, in the same launch, tout [tc, Tpad] bf16 = txᵀ of tx [T, tc] bf16 (row stride ld_tx,
 * 16-byte aligned rows), zero in columns T..Tpad-1: the bytes of mxfp8_transpose_pad(tx, T, tc, ld_tx, tout,
 * Tpad), computed by workgroups of its own after the quantizer's.  The backward's first read of dy (mx_quant(dy2)
 * and dxd, /root/reference/scripts/fused_mlp.py:309-313) with the transposed copy of the saved xs (:291) that the
 * backward kernel takes as a matrix-instruction operand (see mxfp8_transpose_pad).  tc in {16, 32, 64}.
 */
int mxfp8_quant_lora_tp(const void* x, int64_t T, int64_t K, int64_t ld_x, void* q, void* s, const void* w, int64_t rp,
                        float scale, void* out, void* outT, int64_t Tpad, const void* tx, int64_t ld_tx, int64_t tc,
                        void* tout, void* stream);

/*
 * out = bf16(x + bf16(y + scale * xa · Bᵀ)): x, y, out [T, N] bf16 (row stride N), xa [T, r] bf16 (row stride
 * ld_xa), B [N, r] bf16.  The LoRA-B addmm_ and the residual add of o_proj / out_proj in one pass; replaces res_lora /
 * _res_lora_kernel (/root/reference/scripts/mxfp8.py:265-293).  N % 128 == 0, r in {16, 32}, T * N < 2^31; x, y,
 * B, out 16-byte aligned, xa at any element offset and row stride.
 */
int mxfp8_res_lora(const void* x, const void* y, const void* xa, int64_t ld_xa, const void* b, int64_t T, int64_t N,
                   int64_t r, float scale, void* out, void* stream);

/*
 * h[i] = bf16(silu(g[i]) * u[i]) over n bf16 values (n % 8 == 0, 16-byte aligned), silu(g) = g * sigmoid(g) with the
 * sigmoid of the fused MLP kernels.  Replaces _SWIGLU, the compiled silu(g) * u of the unfused MLP path
 * (/root/reference/scripts/shared_prefix.py:172-197).
 */
int mxfp8_swiglu(const void* g, const void* u, int64_t n, void* h, void* stream);

/* Backward of mxfp8_swiglu: du = bf16(dh * silu(g)), dg = bf16(dh * u * sig * (g * (1 - sig) + 1)). */
int mxfp8_swiglu_bwd(const void* g, const void* u, const void* dh, int64_t n, void* dg, void* du, void* stream);

/* Row chunks mxfp8_lora_bwd uses for dy [T, N] (part_db holds chunks * N * r floats); 0 for invalid sizes. */
int64_t mxfp8_lora_bwd_chunks(int64_t T, int64_t N);

/*
 * One read of dy [T, N] bf16 (row stride ld_dy) for the backward of a LoRA-carrying MX linear; replaces lora_bwd /
 * _lora_bwd_kernel / _sum_parts (/root/reference/scripts/mxfp8.py:202-262).
 *  - q != NULL: MX-quantize dy into columns col_tile_off*128 .. + N of the row-major code buffer q (row stride
 *    ld_q) and its blocked scales s (s_col_tiles 128-column tiles per row, ceil(T/128) row tiles; padded rows
 *    scale 0): byte for byte mxfp8_quant_rows(dy) placed at that column offset.
 *  - xa != NULL: dxa [T, r] bf16 (row stride ld_dxa) = bf16(scale * dy · B) and db [N, r] fp32 = scale * dyᵀ · xa,
 *    xa [T, r] bf16 (row stride ld_xa, 16-byte aligned), B [N, r] bf16.  part_dxa: (N/128) * T * r floats,
 *    part_db: mxfp8_lora_bwd_chunks(T, N) * N * r floats of scratch, added in a fixed order (deterministic).
 * N % 128 == 0, r in {16, 32}; at least one of q, xa.
 */
int mxfp8_lora_bwd(const void* dy, int64_t T, int64_t N, int64_t ld_dy, void* q, int64_t ld_q, void* s,
                   int64_t s_col_tiles, int64_t col_tile_off, const void* xa, int64_t ld_xa, const void* b, int64_t r,
                   float scale, void* dxa, int64_t ld_dxa, float* db, float* part_dxa, float* part_db, void* stream);

/*
 * One layer of mxfp8_lora_bwd_batch: dy [T, N] bf16 (row stride ld_dy), its codes at column tile col_tile_off of the
 * batch's code buffer, xa [T, r] (row stride ld_xa), B [N, r], scale, and the outputs and scratch of
 * mxfp8_lora_bwd: dxa [T, r] bf16 (row stride ld_dxa), db [N, r] fp32, part_dxa (N/128) * T * r floats, part_db
 * mxfp8_lora_bwd_batch_chunks(T, ΣN) * N * r floats.
 */
typedef struct {
  const void* dy;
  int64_t N, ld_dy, col_tile_off;
  const void* xa;
  int64_t ld_xa;
  const void* b;
  float scale;
  void* dxa;
  int64_t ld_dxa;
  float* db;
  float* part_dxa;
  float* part_db;
} mxfp8_lora_bwd_job;

#define MXFP8_LORA_BWD_MAX_JOBS 8

/* Row chunks of every job of mxfp8_lora_bwd_batch for T tokens and ΣN columns over the jobs; 0 if invalid. */
int64_t mxfp8_lora_bwd_batch_chunks(int64_t T, int64_t n_total);

/*
 * mxfp8_lora_bwd of every layer of a group in one launch, plus one launch of their partial sums: the layers'
 * dy stream side by side, with one row chunking for all (mxfp8_lora_bwd_batch_chunks(T, ΣN)).  q / s (or NULL)
 * as in mxfp8_lora_bwd, shared by the jobs.  Replaces the per-layer lora_bwd calls of the grouped backward
 * (/root/reference/scripts/fused_linear.py:219-259).  n_jobs <= MXFP8_LORA_BWD_MAX_JOBS, r in {16, 32}.
 * d(xa) is the same bits as mxfp8_lora_bwd's; dB is summed over other row chunks (fp32 rounding).
 */
int mxfp8_lora_bwd_batch(const mxfp8_lora_bwd_job* jobs, int64_t n_jobs, int64_t T, int64_t r, void* q, int64_t ld_q,
                         void* s, int64_t s_col_tiles, void* stream);

/*
 * out [C, Tpad] bf16 = xᵀ of x [T, C] bf16 (row stride ld_x, 16-byte aligned rows), zero in columns T..Tpad-1.
 * No counterpart in the reference, which saves xs = x·Sᵀ for the backward (/root/reference/scripts/
 * fused_mlp.py:291) and reads it row-wise: here the backward kernel takes xsᵀ as a matrix-instruction operand,
 * so the backward rebuilds it from the saved xs.  C in {16, 32, 64}.
 */
int mxfp8_transpose_pad(const void* x, int64_t T, int64_t C, int64_t ld_x, void* out, int64_t Tpad, void* stream);

/*
 * One copy of mxfp8_pack_bf16: for r < rows, c < cols, dst[r * dst_ld + c] (transpose == 0) or
 * dst[c * dst_ld + r] (transpose != 0) = bf16(src[r * src_ld + c]), rounded to nearest even (NaN stays NaN);
 * src fp32 (src_f32 != 0) or bf16, or NULL for zeros.  dst is bf16.
 */
typedef struct {
  const void* src;
  int64_t src_ld;
  int64_t src_f32;
  int64_t rows, cols;
  void* dst;
  int64_t dst_ld;
  int64_t transpose;
} mxfp8_pack_job;

#define MXFP8_PACK_MAX_JOBS 32

/*
 * The n_jobs copies of jobs[] (host memory, n_jobs <= MXFP8_PACK_MAX_JOBS) in ONE launch; the destinations of
 * one call must not overlap.  Replaces the per-step bf16 casts and concatenations of the LoRA weights of a
 * layer group (/root/reference/scripts/fused_linear.py:55-62, :88-101: B.to(dt), torch.cat of the A rows, and
 * here also S zero-padded to the rank the kernels take, its transpose and the block-diagonal B of the group's
 * one forward GEMM), which the reference makes with one torch operation each.
 */
int mxfp8_pack_bf16(const mxfp8_pack_job* jobs, int64_t n_jobs, void* stream);

/*
 * The gate|up MX GEMM with the SwiGLU forward fused into its epilogue: one launch replacing
 * torch._scaled_mm(q, hold.w) + _fwd_kernel (/root/reference/scripts/fused_mlp.py:279-282, :65-109):
 *   gu = bf16(MX(x) · W_guᵀ) [M, 2N] (gate | up, the tensor the forward saves) in the fused-tile layout;
 *   g = bf16(gu_g + s_g · xs_g·B_gᵀ), u = bf16(gu_u + s_u · xs_u·B_uᵀ), h = bf16(g / (exp(-g) + 1) · u);
 *   MX(h) -> q_h (MX-tiled, [ceil(M/16)*16, N]) and s_h (blocked, ceil(M/128) tile rows; padded rows 0);
 *   part [2N/128, M, r] fp32: each output tile's xS_down = h · A_dᵀ over its 64 columns (add them in order).
 * a / sa: MX-tiled codes and blocked scales of x [M, K]; b / sb: W_gu [2N, K] in the fused row order (output
 * tile t holds gate columns 64t..64t+63 then up columns 64t..64t+63, each 32-row block permuted by
 * pi_col(a) = ((a >> 2) & 1) * 16 + (a >> 3) * 4 + (a & 3)), MX-tiled, with its blocked scales.  xs [M, 2r],
 * bg, bu [N, r], ad [r, N] bf16.  N % 128 == 0, K % 128 == 0, r in {16, 32}, M * 2N < 2^31.
 */
int mxfp8_gemm_swiglu_fwd(const void* a, const void* sa, const void* b, const void* sb, int64_t M, int64_t N, int64_t K,
                          const void* xs, const void* bg, const void* bu, const void* ad, int64_t r, float s_g,
                          float s_u, void* gu, void* q_h, void* s_h, float* part, void* stream);

/*
 * The dgrad GEMM of h with the SwiGLU backward fused into its epilogue: one launch replacing
 * torch._scaled_mm(MX(dy), W_down) + _bwd_kernel (/root/reference/scripts/fused_mlp.py:307-314, :112-175):
 *   dhm = bf16(MX(dy) · W_down) [M, N] stays in registers (it is never stored);
 *   g, u, h recomputed from gu as in the forward; dh = bf16(dhm + dxd · A_dᵀ); du = bf16(dh · silu(g)),
 *   dg = bf16(dh · u · σ(g) · (1 + g (1 - σ(g))));
 *   MX(dg) | MX(du) -> q (MX-tiled, [ceil(M/16)*16, 2N], dg at columns 0..N-1, du at N..2N-1) and s (blocked,
 *   ceil(M/128) tile rows; padded rows 0);
 *   dxa_part [N/128, M, 3r]: each 128-column tile's dg · B_g | du · B_u | h · A_dᵀ (add them in order; the same
 *   bits as mxfp8_mlp_bwd with CG = 128);
 *   dbg_part, dbu_part [ceil(M/256), N, r] and dad_part [ceil(M/256), r, N]: each 256-row tile row's dgᵀ · xs_g,
 *   duᵀ · xs_u and dxdᵀ · h (add them in order).
 * a / sa: MX-tiled codes and blocked scales of dy [M, K]; b / sb: W_downᵀ [N, K] with each 32-row block in the
 * dgrad row order (row a holds logical row pi_col(a), as in mxfp8_gemm_swiglu_fwd), MX-tiled, with its blocked
 * scales.  gu [ceil(M/32)*32, 2N] in the fused-tile layout (mxfp8_gemm_swiglu_fwd's output); xs [M, 2r] and its
 * transpose xsT [2r, Tpad]; dxd [M, r] = bf16(bf16(dy · B_d) · s_d) and dxdT [r, Tpad] (Tpad = ceil(M/128)*128,
 * zero past M: mxfp8_quant_lora's outputs); bg, bu [N, r], adT [N, r] and their transposes bgT, buT, ad [r, N],
 * bf16.  N % 128 == 0, K % 128 == 0, r == 16, M * 2N < 2^31.
 */
int mxfp8_gemm_swiglu_bwd(const void* a, const void* sa, const void* b, const void* sb, int64_t M, int64_t N, int64_t K,
                          const void* gu, const void* xs, const void* xsT, const void* dxd, const void* dxdT,
                          const void* bg, const void* bgT, const void* bu, const void* buT, const void* ad,
                          const void* adT, int64_t r, float s_g, float s_u, void* q, void* s, float* dxa_part,
                          float* dbg_part, float* dbu_part, float* dad_part, void* stream);

/* Token chunks mxfp8_lora_tn uses for [T, K] (its partial buffer holds chunks * rp * K floats). */
int64_t mxfp8_lora_tn_chunks(int64_t T, int64_t K);

/*
 * out = bf16(Σ_t p[t, ρ] x[t, k]) (then bf16(· scale) when scale != 1) over the T tokens, as [rp, K]
 * (transpose = 0) or [K, rp] (transpose = 1), fp32 holding the bf16 value (out_f32 = 1) or bf16; x [T, K],
 * p [T, rp] bf16; part: scratch of mxfp8_lora_tn_chunks(T, K) * rp * K floats, the per-chunk sums (added in
 * chunk order).  Replaces dB_d = (dy2.t() @ xS_down).mul_(s_d) and dA = dxa.t() @ x2
 * (/root/reference/scripts/fused_mlp.py:316-318, :333).  K % 128 == 0, rp in {16, 32, 64}.
 */
int mxfp8_lora_tn(const void* x, int64_t T, int64_t K, int64_t ld_x, const void* p, int64_t rp, int64_t chunks,
                  float* part, float scale, int64_t transpose, int64_t out_f32, void* out, void* stream);

/* One token reduction of mxfp8_lora_tn_batch: out = bf16(Σ_t p[t, ρ] x[t, k]) (then bf16(· scale)), as in
 * mxfp8_lora_tn with the same arguments. */
typedef struct {
  const void* x;     /* [T, K] bf16, row stride ld_x (>= K, a multiple of 8), 16-byte aligned */
  int64_t ld_x;
  const void* p;     /* [T, rp] bf16, 16-byte aligned */
  int64_t rp;        /* 16, 32 or 64 */
  float scale;
  int64_t transpose; /* out [rp, K] (0) or [K, rp] (1) */
  int64_t out_f32;   /* out holds fp32 values of the bf16 result (1) or bf16 (0) */
  void* out;
} mxfp8_lora_tn_job;

#define MXFP8_LORA_TN_MAX_JOBS 4

/*
 * Up to MXFP8_LORA_TN_MAX_JOBS token reductions over the same T tokens and K columns in one launch, and their
 * chunk sums in one more: every job's result is bit for bit mxfp8_lora_tn's with the same chunks.  part: scratch
 * of chunks * (Σ rp over the jobs) * K floats (job j's partials after those of jobs 0..j-1).  Replaces the
 * backward's dB_d = (dy2.t() @ xS_down).mul_(s_d) and dA = dxa.t() @ x2 (/root/reference/scripts/
 * fused_mlp.py:316-318, :333), which both read a [T, K] activation after the backward kernel's sums.
 */
int mxfp8_lora_tn_batch(const mxfp8_lora_tn_job* jobs, int64_t n_jobs, int64_t T, int64_t K, int64_t chunks,
                        float* part, void* stream);

/*
 * mxfp8_gemm_nt (4-wave shape, rank-16, 32 or 48 LoRA epilogue, no workspace) and mxfp8_lora_tn_batch in one
 * launch plus the batch's sums: the token reductions run in workgroups numbered after every GEMM tile, so the
 * dispatcher starts them only once each tile has started, in the workgroup slots the GEMM's last round of tiles
 * leaves idle.  Results bit for bit those of the two calls one after the other (jobs, T_tn, K_tn, chunks and part
 * as in mxfp8_lora_tn_batch).  The jobs must not read c.  Replaces, in the MLP backward, the dx GEMM with its
 * dxa·S addmm_ and the token GEMMs dB_d, dA (/root/reference/scripts/fused_mlp.py:331, :316-318, :333), and in
 * the grouped linears' backward the dx GEMM with its dS·S addmm_ and dA = dSᵀ·x2 (fused_linear.py:269, :271), which
 * the reference runs as separate kernels.  r in {16, 32, 48}, layout without MXFP8_GEMM_WIDE, M > 0.
 */
int mxfp8_gemm_nt_tn(const void* a, const void* sa, int64_t lda, const void* b, const void* sb, int64_t ldb,
                     int64_t M, int64_t N, int64_t K, void* c, int64_t ldc, const void* lora_p, int64_t ld_p,
                     const void* lora_q, int64_t ld_q, int64_t r, float alpha, int64_t layout,
                     const mxfp8_lora_tn_job* jobs, int64_t n_jobs, int64_t T_tn, int64_t K_tn, int64_t chunks,
                     float* part, void* stream);

/*
 * mxfp8_gemm_nt (4-wave shape, rank-16 LoRA epilogue, no workspace) whose epilogue operand P is summed in the same
 * launch: P [M, r] (lora_p, row stride r, written) = bf16(part_scale · Σ_p part[p]) over the n_parts fp32 partials
 * part [n_parts, M, r], p ascending, exactly as mxfp8_sum_parts computes it.  Workgroups numbered before the
 * GEMM's tiles compute P and publish each block of rows; a tile waits for its rows only at its epilogue.  A tile
 * whose wait runs past wait_limit polls sums its own rows of P from part instead (the same bits); wait_limit < 0
 * takes the default, 0 makes every tile do so (for tests).  Results bit for bit those of mxfp8_sum_parts then
 * mxfp8_gemm_nt.  Replaces, in the MLP forward, part.sum(0) of the xS_down partials and the down projection's
 * _scaled_mm + addmm_ (/root/reference/scripts/fused_mlp.py:214, :283-284), separate kernels there.  r must be 16,
 * M > 0, M · r ≤ 2^26; part and lora_p 16-byte aligned.  Launches that overlap on one GPU stay correct but may
 * fall back to the per-tile sums.  On a stream under graph capture it records mxfp8_sum_parts and then
 * mxfp8_gemm_nt, two launches (a replayed launch would repeat the id its flags are matched against).
 */
int mxfp8_gemm_nt_sum(const void* a, const void* sa, int64_t lda, const void* b, const void* sb, int64_t ldb,
                      int64_t M, int64_t N, int64_t K, void* c, int64_t ldc, const float* part, int64_t n_parts,
                      float part_scale, void* lora_p, const void* lora_q, int64_t ld_q, int64_t r, float alpha,
                      int64_t layout, int64_t wait_limit, void* stream);

/*
 * Allocation-free variant of mxfp8_lora_tn: same arguments without `chunks` / `part`, same result bit for bit as
 * mxfp8_lora_tn(..., chunks = mxfp8_lora_tn_noalloc_chunks(T, K, rp), ...).  No counterpart in the reference; it
 * is for callers that cannot allocate device memory (code under HIP graph capture, tight serving or training
 * loops, harnesses that forbid hipMalloc): the chunk partials live in a static 16 MiB device array of the
 * library, one per GPU, held until the process ends, so nothing here allocates or frees.  Limit: rp * K * 4 bytes
 * must fit in it (K <= 65536 at rp = 64); the chunk count is capped so that chunks * rp * K * 4 <= 16 MiB.
 * Every call on one GPU shares that GPU's array: calls that overlap on one GPU (other streams, other threads)
 * race and must be serialized by the caller.  Returns MXFP8_ERR_ARG when the sizes do not fit.
 */
int mxfp8_lora_tn_noalloc(const void* x, int64_t T, int64_t K, int64_t ld_x, const void* p, int64_t rp, float scale,
                          int64_t transpose, int64_t out_f32, void* out, void* stream);

/* Chunk count mxfp8_lora_tn_noalloc uses for [T, K] at rank rp (0 for bad sizes). */
int64_t mxfp8_lora_tn_noalloc_chunks(int64_t T, int64_t K, int64_t rp);

/*
 * The backward kernel's partial sums, added in order, scaled and cast as the reference's backward does
 * (/root/reference/scripts/fused_mlp.py:258, :319-326): dxa [T, 2r] bf16 = bf16(s_g · Σ dxa_g | s_u · Σ dxa_u),
 * xsd [T, r] bf16 = bf16(Σ xS_down), dB_g, dB_u [N, r] fp32 = s · Σ, dA_d [r, N] fp32 = Σ.  Partials as written by
 * mxfp8_mlp_bwd (ncg column groups, nsb super-blocks).
 */
int mxfp8_mlp_bwd_finish(const float* dxa_part, const float* dbg_part, const float* dbu_part, const float* dad_part,
                         int64_t ncg, int64_t nsb, int64_t T, int64_t N, int64_t r, float s_g, float s_u, void* dxa,
                         void* xsd, float* dbg, float* dbu, float* dad, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MXFP8_MLP_H */
