/*
 * trnsparse_hip.h — C ABI of the MI355X (gfx950) trnsparse compute path.
 *
 * This is the drop-in boundary that replaces the reference's device seam:
 * the `nki_*` entry points that `trnsparse/ops.py` lazily imports when the
 * accelerator backend is active (trnsparse/nki/dispatch.py). Every function
 *   - takes plain device pointers, sizes and dtype codes (no torch types),
 *   - launches asynchronously on the caller's HIP stream (`stream`, a
 *     hipStream_t passed as void*; NULL = the default stream),
 *   - never allocates or frees caller memory and keeps no pointer after it
 *     returns (workspace, when needed, is passed in by the caller),
 *   - returns TSP_OK (0) or a negative status; the message of the last
 *     failure on the calling thread is available from tsp_last_error().
 * No C++ exception crosses this boundary.
 *
 * Structure arrays (row pointers, column indices) use int64 like the
 * reference's torch.long tensors (trnsparse/formats.py); CSR entry points
 * also accept int32 via `index_type`.
 */
#ifndef TRNSPARSE_HIP_H
#define TRNSPARSE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ---------------------------------------------------- */
#define TSP_OK 0
#define TSP_EINVAL (-1)       /* bad argument (shape, pointer, alignment)   */
#define TSP_EUNSUPPORTED (-2) /* valid request this library does not serve  */
#define TSP_EHIP (-3)         /* a HIP runtime call or kernel launch failed */

/* ---- element type codes ---------------------------------------------- */
#define TSP_F32 0
#define TSP_F64 1
#define TSP_BF16 2

/* ---- index type codes (CSR) ------------------------------------------ */
#define TSP_I32 0
#define TSP_I64 1

/* Library version as 100*major + minor. */
int tsp_version(void);

/* Message of the last failing call on this thread ("" if none). */
const char* tsp_last_error(void);

/* ======================================================================
 * Block-sparse (BSR) x dense:  C[m, ncols] = A_bsr[m, n] @ B[n, ncols]
 *
 * Replaces nki_bsr_spmm / _BSRSpMMFunction forward
 * (trnsparse/nki/dispatch.py:372-381, :304-328) and the torch spec
 * _bsr_spmm_pytorch (trnsparse/ops.py:162-192).
 *
 * blocks            (n_blocks, block_size, block_size), row-major, `dtype`
 * block_row_ptrs    (ceil(m/block_size)+1,) int64
 * block_col_indices (n_blocks,) int64
 * B                 (n, ncols) with row stride ldb (elements), `dtype`
 * C                 (m, ncols) with row stride ldc, `out_dtype`; every
 *                   element is written (no pre-zeroing needed)
 * row_order         optional (ceil(m/block_size),) int32 permutation of the
 *                   block rows, heaviest first (see tsp_bsr_row_order);
 *                   only changes scheduling, never results. NULL = natural.
 * dtype/out_dtype   TSP_F32/TSP_F32, TSP_BF16/{TSP_BF16,TSP_F32},
 *                   TSP_F64/TSP_F64. Accumulation is fp32 (fp64 for F64).
 * ==================================================================== */
int tsp_bsr_spmm(const void* blocks, int dtype,
                 const int64_t* block_row_ptrs, const int64_t* block_col_indices,
                 int64_t n_blocks, int64_t block_size, int64_t m, int64_t n,
                 const void* B, int64_t ldb, int64_t ncols,
                 void* C, int64_t ldc, int out_dtype,
                 const int32_t* row_order, void* stream);

/* Heaviest-first ordering of block rows (counting sort by stored blocks per
 * row, computed on the device). `order` receives n_block_rows int32. It is
 * a scheduling plan for tsp_bsr_spmm, a property of the sparsity pattern
 * only, and may be cached with it. */
int tsp_bsr_row_order(const int64_t* block_row_ptrs, int64_t n_block_rows,
                      int32_t* order, void* stream);

/* ======================================================================
 * BSR times one vector, fused with a solver's vector update:
 *   out[r] = alpha * (A_bsr x)[r] + beta * u[r] + gamma * v[r] + delta * w[r]
 * for r < m; u, v, w (m,) are optional (NULL: term skipped). x (n,) is
 * read as zero past n. out may alias u, v or w but not x. dtype of blocks,
 * x, u, v, w and out: TSP_F32 / TSP_F64 / TSP_BF16 (fp32 accumulation, fp64
 * for F64). row_order: optional heaviest-first block-row permutation.
 * Replaces bsr_spmm with N = 1 (trnsparse/ops.py:162-192 as the reference's
 * solvers call it, trnsparse/iterative.py:44-50) and the update statements
 * of richardson_bsr / chebyshev_bsr (iterative.py:256-295, 200-253).
 * ==================================================================== */
int tsp_bsr_spmv(const void* blocks, int dtype, const int64_t* block_row_ptrs,
                 const int64_t* block_col_indices, int64_t n_blocks,
                 int64_t block_size, int64_t m, int64_t n, const void* x,
                 double alpha, const void* u, double beta, const void* v,
                 double gamma, const void* w, double delta, void* out,
                 const int32_t* row_order, void* stream);

/* ======================================================================
 * Backward of C = A_bsr @ B.
 *
 * Replaces the backward of _BSRSpMMFunction
 * (trnsparse/nki/dispatch.py:331-369: dA_k = dC_i B_j^T on the stored
 * pattern, dB = A_dense^T dC), which gathers dense panels on the host.
 *
 * tsp_bsr_sddmm: grad_blocks[k] = G[rows of block row i_k] @ B[rows of block
 *   column j_k]^T for every stored block k (rows past m of G and past n of B
 *   count as zero); the SDDMM restricted to the pattern.
 *   G            (m, ncols) row stride ldg (dC)
 *   B            (n, ncols) row stride ldb
 *   block_rows   (n_blocks,) int64 block row of each stored block
 *   block_col_indices (n_blocks,) int64
 *   grad_blocks  (n_blocks, block_size, block_size) row-major, every element
 *                written. dtype TSP_F32 / TSP_F64 / TSP_BF16 for G, B and
 *                grad_blocks (fp32 accumulation, fp64 for F64).
 *
 * tsp_bsr_spmm_t: out[n, ncols] = A_bsr^T @ X over the block-column view of
 *   the pattern. col_ptrs (n_block_cols+1,) int64 with n_block_cols =
 *   ceil(n/block_size); col_block_ids / col_block_rows (n_blocks,) int64 give,
 *   column by column in increasing block-row order, the stored block index and
 *   its block row (the sums run in that order). X is (m, ncols) row stride
 *   ldx (rows past m count as zero); out (n, ncols) row stride ldo, every
 *   element written. col_order: optional heaviest-first permutation of the
 *   block columns (tsp_bsr_row_order on col_ptrs), scheduling only.
 * ==================================================================== */
/* tsp_bsr_col_view: the pattern views the two backward kernels take, built
 *   on the device from the block CSR (block_row_ptrs (n_block_rows+1,),
 *   block_col_indices (nnzb,), int64): block_rows (nnzb,) the block row of
 *   every stored block; col_ptrs (n_block_cols+1,); col_block_ids /
 *   col_block_rows (nnzb,), per block column in increasing block-row order,
 *   the stored block index and its block row (a stable sort of the blocks
 *   by column). The reference backward gathers dense panels on the host
 *   instead (trnsparse/nki/dispatch.py:348-369); this view replaces that
 *   gather. nnzb, n_block_rows <= 2^32. workspace:
 *   tsp_bsr_col_view_workspace_size(nnzb, n_block_cols) bytes. */
int64_t tsp_bsr_col_view_workspace_size(int64_t nnzb, int64_t n_block_cols);
int tsp_bsr_col_view(const int64_t* block_row_ptrs,
                     const int64_t* block_col_indices, int64_t n_block_rows,
                     int64_t n_block_cols, int64_t nnzb, int64_t* block_rows,
                     int64_t* col_ptrs, int64_t* col_block_ids,
                     int64_t* col_block_rows, void* workspace,
                     int64_t workspace_bytes, void* stream);
int tsp_bsr_sddmm(const void* G, int64_t ldg, int64_t m,
                  const void* B, int64_t ldb, int64_t n, int64_t ncols,
                  const int64_t* block_rows, const int64_t* block_col_indices,
                  int64_t n_blocks, int64_t block_size, int dtype,
                  void* grad_blocks, void* stream);

/* tsp_bsr_sddmm_ex: tsp_bsr_sddmm with the blocks written in out_dtype:
 *   out_dtype == dtype is tsp_bsr_sddmm itself; dtype TSP_BF16 with
 *   out_dtype TSP_F32 keeps the fp32 accumulators (block_size 128, ncols,
 *   ldg, ldb multiples of 8, 16-byte aligned G and B). The block scores of
 *   the block-sparse attention path (S = Q K^T, dP = dO V^T on the mask
 *   pattern) are formed this way before their fp32 softmax; the reference
 *   forms them per block inside its attention loops
 *   (trnsparse/ops.py:311, 349, 462, 466). */
int tsp_bsr_sddmm_ex(const void* G, int64_t ldg, int64_t m,
                     const void* B, int64_t ldb, int64_t n, int64_t ncols,
                     const int64_t* block_rows,
                     const int64_t* block_col_indices, int64_t n_blocks,
                     int64_t block_size, int dtype, void* out_blocks,
                     int out_dtype, void* stream);

int tsp_bsr_spmm_t(const void* blocks, int dtype,
                   const int64_t* col_ptrs, const int64_t* col_block_ids,
                   const int64_t* col_block_rows, int64_t n_block_cols,
                   int64_t block_size, int64_t m, int64_t n,
                   const void* X, int64_t ldx, int64_t ncols,
                   void* out, int64_t ldo, const int32_t* col_order,
                   void* stream);

/* ======================================================================
 * CSR sparse x dense (bandwidth-bound; no MFMA)
 *
 * Replaces the reference's spmv (trnsparse/ops.py:30-48, torch
 * sparse_csr @ x) and spmm (ops.py:51-78; NKI nki_spmm,
 * trnsparse/nki/dispatch.py:181-190, which densified A):
 *   out = alpha * (A @ x)  [+ beta * y  when y != NULL and beta != 0]
 * values (nnz,) `dtype` (TSP_F32 or TSP_F64, accumulated in that type),
 * col_indices (nnz,) and row_ptrs (m+1,) both `index_type`.
 * ==================================================================== */

/* Number of int64 entries of the SpMV work-partition table for an m-row
 * matrix with nnz stored entries (<0 on bad sizes). */
int64_t tsp_csr_plan_size(int64_t m, int64_t nnz);

/* Build the SpMV work-partition table (`windows`, tsp_csr_plan_size
 * entries) from row_ptrs on the device. Depends only on the pattern. */
int tsp_csr_plan(const void* row_ptrs, int index_type, int64_t m, int64_t nnz,
                 int64_t* windows, void* stream);

/* ---- length-bucketed SpMV (the same result as tsp_csr_spmv) ----------
 * Row-per-wavefront kernels with the skewed rows split out: rows with at
 * most 32 entries take 8 lanes each in natural order, rows with up to 2048
 * one wavefront each, longer rows one 512-thread workgroup each (lists in
 * the plan). tsp_csr_bucket_plan_size(m) bytes of plan (int32: the medium
 * and long row counts at [0] and [1], the lists from [4] and [4 + m]),
 * built by tsp_csr_bucket_plan from the pattern; the caller reads the two
 * counts back once and passes them to tsp_csr_bucketed_spmv. Same
 * reference interface as tsp_csr_spmv (trnsparse/ops.py:30-48). */
int64_t tsp_csr_bucket_plan_size(int64_t m);

int tsp_csr_bucket_plan(const void* row_ptrs, int index_type, int64_t m,
                        void* plan, void* stream);

int tsp_csr_bucketed_spmv(const void* values, int dtype,
                          const void* col_indices, const void* row_ptrs,
                          int index_type, int64_t m, int64_t n, int64_t nnz,
                          const void* plan, int64_t n_medium, int64_t n_long,
                          const void* x, double alpha, const void* y,
                          double beta, void* out, void* stream);

/* out (m,) = alpha * A @ x (+ beta * y); x (n,), y (m,) or NULL. */
int tsp_csr_spmv(const void* values, int dtype, const void* col_indices,
                 const void* row_ptrs, int index_type, int64_t m, int64_t n,
                 int64_t nnz, const int64_t* windows, const void* x,
                 double alpha, const void* y, double beta, void* out,
                 void* stream);

/* ---- SpMV over a cached column-sorted plan (fp32 values) -------------
 * Same result as tsp_csr_spmv (reference trnsparse/ops.py:30-48, the
 * torch.sparse_csr @ x call at :45), computed from a reordered copy of the
 * matrix built once per pattern: tiles of 2^rbits rows x 2^cbits columns,
 * each tile's entries sorted by column, 8 bytes per entry (packed row /
 * column within the tile and the value), so the x gathers of one wavefront
 * instruction share cache lines.
 *
 * Row sums are exact int64 fixed-point sums of the fp32 products v * x:
 * the plan keeps v * 2^(61 - e_r) with sum_j |v_rj| < 2^e_r per row, x is
 * scaled by 2^-e_x with max |x| < 2^e_x, each product is rounded to an
 * integer (exact when its magnitude is at least 2^23 units) and added in
 * LDS. Integer sums do not depend on the order of the additions, so
 * repeated calls are bit-identical; the result is the exactly rounded sum
 * of the fp32 products of the reference, up to one rounding per column
 * group. A row is summed from the CSR arrays instead (fp32 products in CSR
 * order, fp64 sum) when x holds inf or NaN, when the row holds a
 * non-finite value or values spread over more than ~2^180, or when one of
 * its products was rounded and the row's result is below cnt * 2^23 units
 * (so the rounding could exceed 2^-24 of it). The result can differ from
 * tsp_csr_spmv in the last bits.
 *
 * geometry (10 int64, host memory), filled by tsp_csr_colplan_geometry:
 *   [0] rbits   [1] row blocks   [2] cbits   [3] column groups G
 *   [4] tiles   [5] sort key bits [6] plan bytes  [7] build workspace bytes
 *   [8] SpMV workspace bytes  [9] padded entries
 * rows_per_block_log2 (12..14) and tiles_hint tune the tiling; 0 = auto.
 * TSP_EUNSUPPORTED when nnz > 2^32 - 2. The plan holds each entry's
 * position k in the pattern (uint32) and row_ptrs[0] (any value) beside
 * them; tsp_csr_colplan_refresh reads values[row_ptrs[0] + k]. */
int tsp_csr_colplan_geometry(int64_t m, int64_t n, int64_t nnz,
                             int rows_per_block_log2, int64_t tiles_hint,
                             int64_t* geometry);

/* Build the plan (geometry[6] bytes at `plan`, device) from the CSR arrays;
 * `workspace` (geometry[7] bytes, device) is scratch for the build only. */
int tsp_csr_colplan_build(const void* values, int dtype,
                          const void* col_indices, const void* row_ptrs,
                          int index_type, int64_t m, int64_t n, int64_t nnz,
                          const int64_t* geometry, void* plan,
                          void* workspace, void* stream);

/* Copy new values of the same pattern into the plan (the row exponents from
 * row_ptrs, then one gather pass). */
int tsp_csr_colplan_refresh(const void* values, int dtype,
                            const void* row_ptrs, int index_type, int64_t m,
                            int64_t n, int64_t nnz, const int64_t* geometry,
                            void* plan, void* stream);

/* out (m,) = alpha * A @ x (+ beta * y) over the plan; x (n,), y (m,) or
 * NULL; values / col_indices / row_ptrs: the CSR arrays the plan was built
 * (or last refreshed) from, read only for the rows summed from them;
 * workspace: geometry[8] bytes of device memory. */
int tsp_csr_colplan_spmv(const void* plan, int dtype, int64_t m, int64_t n,
                         int64_t nnz, const int64_t* geometry,
                         const void* values, const void* col_indices,
                         const void* row_ptrs, int index_type, const void* x,
                         double alpha, const void* y, double beta, void* out,
                         void* workspace, void* stream);

/* out (m, ncols; row stride ldo) = alpha * A @ B (+ beta * C);
 * B (n, ncols; stride ldb), C (m, ncols; stride ldc) or NULL. */
int tsp_csr_spmm(const void* values, int dtype, const void* col_indices,
                 const void* row_ptrs, int index_type, int64_t m, int64_t n,
                 int64_t nnz, const void* B, int64_t ldb, int64_t ncols,
                 double alpha, const void* C, int64_t ldc, double beta,
                 void* out, int64_t ldo, void* stream);

/* Values gradient of out = alpha * A @ X on A's own pattern (the reference's
 * autograd for spmm, trnsparse/nki/dispatch.py:174-178, forms
 * grad_out @ B^T densely and projects it onto the pattern):
 *   out_values[p] = alpha * sum_c G[row p][c] * X[col p][c],
 * G (m, ncols; stride ldg), X (n, ncols; stride ldx); ncols = 1 with unit
 * strides for the SpMV case. No values argument: only the pattern is read. */
int tsp_csr_sddmm(const void* col_indices, const void* row_ptrs, int index_type,
                  int64_t m, int64_t n, int64_t nnz, const void* G, int64_t ldg,
                  const void* X, int64_t ldx, int64_t ncols, int dtype,
                  double alpha, void* out_values, void* stream);

/* ======================================================================
 * Schwarz-screened dense SpMM:  C = (A * mask) @ B
 *   Q = sqrt(|diag|), mask[i,k] = Q[i]*Q[k] > threshold_sqrt, evaluated in
 *   diag's precision (diag_dtype TSP_F32 or TSP_F64; threshold_sqrt is
 *   rounded to that precision), A (m, m; stride lda) and B (m, ncols;
 *   stride ldb) `dtype` (TSP_F32 on the MFMA path, TSP_F64 generic),
 *   C (m, ncols; stride ldc) written in full.
 * Replaces nki_screened_spmm / _ScreenedSpMMFunction forward
 * (trnsparse/nki/dispatch.py:384-494) and the torch spec
 * (trnsparse/ops.py:262-277). `workspace` holds
 * tsp_screened_workspace_size(m, diag_dtype) bytes (Q and per-tile maxima),
 * 16-byte aligned.
 * ==================================================================== */
int64_t tsp_screened_workspace_size(int64_t m, int diag_dtype);

int tsp_screened_spmm(const void* A, int dtype, int64_t lda, const void* diag,
                      int diag_dtype, double threshold_sqrt, int64_t m,
                      const void* B, int64_t ldb, int64_t ncols, void* C,
                      int64_t ldc, void* workspace, void* stream);

/* tsp_screened_spmm without the workspace argument: no counterpart in the
 * reference. For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc): the
 * workspace lives in a 1 MiB device array of the library, one per GPU, kept
 * until the process ends. m is limited to
 * tsp_screened_spmm_noalloc_max_rows(diag_dtype) rows (a larger m returns
 * TSP_EINVAL). The call allocates and frees nothing. Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (other streams or
 * threads) race; serialize them. Same results as tsp_screened_spmm. */
int64_t tsp_screened_spmm_noalloc_max_rows(int diag_dtype);

int tsp_screened_spmm_noalloc(const void* A, int dtype, int64_t lda,
                              const void* diag, int diag_dtype,
                              double threshold_sqrt, int64_t m,
                              const void* B, int64_t ldb, int64_t ncols,
                              void* C, int64_t ldc, void* stream);

/* Gradients of C = (A * mask) @ B with the same mask:
 *   dA = (dC @ B^T) * mask   (m, m; stride ldda), written when dA != NULL
 *   dB = (A * mask)^T @ dC   (m, ncols; stride lddb), written when dB != NULL
 * dC (m, ncols; stride lddc) in `dtype`; no gradient for diag or the
 * threshold (the mask is discrete). The mask is not materialised: 128x128
 * tile pairs whose largest Q product is at or below the threshold are
 * skipped (dA tiles written as zeros). `workspace` as for
 * tsp_screened_spmm. TSP_F32 runs the MFMA kernels, TSP_F64 the generic
 * ones. Replaces _ScreenedSpMMFunction.backward
 * (trnsparse/nki/dispatch.py:478-484). */
int tsp_screened_spmm_backward(const void* A, int dtype, int64_t lda,
                               const void* diag, int diag_dtype,
                               double threshold_sqrt, int64_t m,
                               const void* B, int64_t ldb, int64_t ncols,
                               const void* dC, int64_t lddc, void* dA,
                               int64_t ldda, void* dB, int64_t lddb,
                               void* workspace, void* stream);

/* ======================================================================
 * Block-sparse attention forward, per head h < n_heads:
 *   O[h] = softmax_rows(scale * Q[h] K[h]^T restricted to the stored mask
 *          blocks) V[h]
 * Q, K, V, O (n_heads, seq_len, head_dim) contiguous, `dtype` (TSP_BF16 and
 * TSP_F32 on the MFMA path for block_size 128, scale > 0 and head_dim 64,
 * 128 or 256, TSP_BF16 also at 512; TSP_F64 and other shapes on the generic
 * path). The mask (block_row_ptrs with at
 * least seq_len/block_size + 1 entries, block_col_indices) is shared by all
 * heads; only its pattern is used. Rows of an empty block row, and rows past
 * (seq_len/block_size)*block_size, are zero.
 * row_max / row_denom (optional, both or neither): (n_heads,
 * seq_len/block_size, block_size) in float (double for TSP_F64) — the row
 * max of the scaled scores and the softmax denominator clamped at 1e-12
 * (0 and 1e-12 for empty rows), saved for the backward pass.
 * Replaces nki_bsr_attn_tiled (trnsparse/nki/dispatch.py:580-677) and the
 * torch spec _block_sparse_attn_pytorch (trnsparse/ops.py:280-357).
 * ==================================================================== */
int tsp_bsa_fwd(const void* Q, const void* K, const void* V, int dtype,
                int64_t n_heads, int64_t seq_len, int64_t head_dim,
                const int64_t* block_row_ptrs, const int64_t* block_col_indices,
                int64_t block_size, double scale, void* O, void* row_max,
                void* row_denom, void* stream);

/* ====================================================================
 * Block-sparse attention as block-sparse products (any head_dim).
 *
 * For the head_dims the one-pass kernels above do not serve (head_dim over
 * 256 except the bf16 forward at 512; bf16 gradients at head_dim 256 and
 * over), attention runs as block-sparse
 * products over the mask stacked over heads: the pattern whose block row
 * h * Mt + i holds the mask blocks of block row i shifted by h * Mt block
 * columns, so Q, K, V (n_heads, seq_len, head_dim) contiguous are its
 * (n_heads * seq_len, head_dim) operands. Block scores S = Q K^T come from
 * tsp_bsr_sddmm_ex (fp32), the softmax below turns them into P, O = P V is
 * tsp_bsr_spmm; the backward forms S and dP = dO V^T the same way, P and
 * dS below, and dV = P^T dO, dK = dS^T Q (tsp_bsr_spmm_t), dQ = dS K
 * (tsp_bsr_spmm). Blocks are (nnzb, 128, 128) fp32 row-major in the stacked
 * pattern's order. Semantics as tsp_bsa_fwd / tsp_bsa_bwd.
 *
 * tsp_bsa_block_softmax: per row r of stacked block row R (row R * 128 + r
 *   of the stacked operands), over the row's entries in blocks
 *   block_row_ptrs[R] .. block_row_ptrs[R + 1] - 1:
 *     row_max[row]   = max scale * S,  row_denom[row] = max(sum exp(scale *
 *     S - row_max), 1e-12)  (0 and 1e-12 for a row with no block)
 *     P              = exp(scale * S - row_max) / row_denom, written in
 *                      out_dtype (TSP_F32 may alias S, TSP_BF16)
 *   Replaces the reference's tile stats, row reduction and weighting
 *   (trnsparse/ops.py:302-351; trnsparse/nki/dispatch.py:562-577).
 * tsp_bsa_block_grad: per stored block k (block row block_rows[k]), with
 *   the forward's stats and Drow[row] = sum_d dO[row][d] O[row][d]:
 *     P  = exp(scale * S - row_max) / row_denom
 *     dS = scale * P * (dP - Drow)
 *   written in out_dtype (TSP_F32 may alias S and dP; TSP_BF16).
 *   Replaces the per-block P and dS of trnsparse/ops.py:461-467.
 * tsp_bsa_rowdot: Drow[r] = sum_d dO[r][d] O[r][d] in fp32 for rows r <
 *   rows of (rows, head_dim) contiguous O and dO in `dtype` (TSP_F32,
 *   TSP_BF16). Replaces trnsparse/ops.py:395.
 * ==================================================================== */
int tsp_bsa_block_softmax(const float* S, const int64_t* block_row_ptrs,
                          int64_t n_block_rows, int64_t block_size,
                          double scale, void* P, int out_dtype,
                          float* row_max, float* row_denom, void* stream);
int tsp_bsa_block_grad(const float* S, const float* dP,
                       const int64_t* block_rows, int64_t n_blocks,
                       int64_t block_size, double scale,
                       const float* row_max, const float* row_denom,
                       const float* Drow, void* P, void* dS, int out_dtype,
                       void* stream);
int tsp_bsa_rowdot(const void* O, const void* dO, int dtype, int64_t rows,
                   int64_t head_dim, float* Drow, void* stream);
/* tsp_bsa_block_pgrad: tsp_bsr_sddmm_ex for S = Q K^T and dP = dO V^T and
 *   tsp_bsa_block_grad in one kernel for bf16 (the fp32 scores stay in
 *   registers): Q, K, V, dO (rows, head_dim) bf16 contiguous, head_dim a
 *   multiple of 8; P and dS written as bf16 blocks. Replaces the per-block
 *   products and P / dS of trnsparse/ops.py:461-467. */
int tsp_bsa_block_pgrad(const void* Q, const void* K, const void* V,
                        const void* dO, int dtype, int64_t rows,
                        int64_t head_dim, const int64_t* block_rows,
                        const int64_t* block_col_indices, int64_t n_blocks,
                        int64_t block_size, double scale,
                        const float* row_max, const float* row_denom,
                        const float* Drow, void* P, void* dS, void* stream);

/* ====================================================================
 * Block-sparse attention backward, per head h < n_heads, from the forward's
 * output O and row stats (row_max, row_denom as tsp_bsa_fwd writes them):
 *   D[q]     = sum_d dO[q][d] O[q][d]
 *   P[q][k]  = exp(scale * Q[q].K[k] - row_max[q]) / row_denom[q]
 *   dS[q][k] = P[q][k] (dO[q].V[k] - D[q])
 *   dQ = scale * dS K,  dK = scale * dS^T Q,  dV = P^T dO
 * over the stored mask blocks of block rows < seq_len/block_size. Q, K, V,
 * O, dO, dQ, dK, dV (n_heads, seq_len, head_dim) contiguous in `dtype`;
 * every element of dQ, dK, dV is written (zero where no stored block
 * reaches). The mask comes in both views: block_row_ptrs /
 * block_col_indices (row view, >= seq_len/block_size + 1 pointers) and
 * col_ptrs[n_block_cols + 1] / col_block_rows (column view: the block rows
 * below seq_len/block_size storing each block column, any order).
 *
 * The column pass runs over a plan made on the host by tsp_bsa_bwd_plan
 * from a host copy of col_ptrs: call it with plan = NULL to get its length
 * (int32 entries), then again with a buffer of that length. Its header
 * holds n_items, n_splits, n_partials; `plan` of tsp_bsa_bwd is a device
 * copy of the whole plan. `workspace` holds
 * tsp_bsa_bwd_workspace_size(n_heads, seq_len, head_dim, n_partials) bytes.
 * block_size 128 with scale > 0 runs on the MFMA kernels for bf16 at
 * head_dim 128 and fp32 at head_dim 64, 128 and 256; other shapes and fp64
 * run on the generic kernels (which ignore the plan).
 * Replaces nki_bsr_attn_bwd (trnsparse/nki/dispatch.py:813-929; its host
 * gathers _attn_bwd_gather, dispatch.py:680-810) and the torch backward
 * _block_sparse_attn_backward (trnsparse/ops.py:360-473).
 * ==================================================================== */
int64_t tsp_bsa_bwd_plan(const int64_t* col_ptrs, int64_t n_block_cols,
                         int64_t n_heads, int64_t seq_len, int64_t block_size,
                         int32_t* plan, int64_t capacity);
int64_t tsp_bsa_bwd_workspace_size(int64_t n_heads, int64_t seq_len,
                                   int64_t head_dim, int64_t n_partials);
int tsp_bsa_bwd(const void* Q, const void* K, const void* V, const void* O,
                const void* dO, int dtype, int64_t n_heads, int64_t seq_len,
                int64_t head_dim, const int64_t* block_row_ptrs,
                const int64_t* block_col_indices, const int64_t* col_ptrs,
                const int64_t* col_block_rows, int64_t n_block_cols,
                int64_t block_size, double scale, const void* row_max,
                const void* row_denom, void* dQ, void* dK, void* dV,
                const int32_t* plan, int64_t n_items, int64_t n_splits,
                int64_t n_partials, void* workspace, void* stream);

/* ====================================================================
 * Format construction on the device (bit-exact structure).
 *
 * Dense inputs are row-major with row stride lda (elements), dtype
 * TSP_F32 / TSP_F64 / TSP_BF16; structure arrays are int64. A threshold
 * compares in the matrix dtype after rounding to it (torch's comparison of
 * a tensor with a Python float).
 *
 * BSR from dense (replaces BSRMatrix.from_dense, trnsparse/formats.py:
 * 183-221), two calls with a host read of the block count between them:
 *   tsp_bsr_from_dense_pattern: keep (ceil(m/b)*ceil(n/b) uint8, row-major
 *     block grid) = [max |v| over the zero-padded block > threshold] (a NaN
 *     makes the block not kept), row_ptrs (ceil(m/b)+1) = cumulative kept
 *     counts; workspace: tsp_format_workspace_size(ceil(m/b)) bytes.
 *   tsp_bsr_from_dense_fill: col_indices (n_blocks = row_ptrs[last]) in
 *     increasing order within each block row, blocks (n_blocks, b, b)
 *     row-major with the padding zero.
 * tsp_bsr_to_dense (replaces BSRMatrix.to_dense, formats.py:233-251):
 *   out (m, n), row stride ldo; each stored block (the last entry of a
 *   repeated one) in place, zeros elsewhere.
 * CSR from dense (replaces formats.from_dense, formats.py:269-278):
 *   tsp_csr_from_dense_pattern: row_ptrs (m+1) of |v| > threshold
 *     (workspace: tsp_format_workspace_size(m) bytes); then
 *   tsp_csr_from_dense_fill: col_indices / values (row_ptrs[m]) in row
 *     order, columns increasing.
 * tsp_csr_to_dense (replaces CSRMatrix.to_dense, formats.py:49-52):
 *   duplicate entries of a row add up in entry order.
 * tsp_csr_row_indices (replaces the row expansion of CSRMatrix.to_coo,
 *   formats.py:54-65): rows[k] = row of entry k.
 * tsp_coo_to_csr (replaces COOMatrix.to_csr, formats.py:104-124): entries
 *   sorted by row*n + col (stable), row_ptrs (m+1); nnz < 2^32 (the device
 *   sort's positions are 32-bit; TSP_EUNSUPPORTED past it); workspace:
 *   tsp_coo_to_csr_workspace_size(nnz, m, n) bytes.
 * ==================================================================== */
int64_t tsp_format_workspace_size(int64_t rows);
int tsp_bsr_from_dense_pattern(const void* A, int dtype, int64_t lda, int64_t m,
                               int64_t n, int64_t block_size, double threshold,
                               uint8_t* keep, int64_t* row_ptrs,
                               void* workspace, void* stream);
int tsp_bsr_from_dense_fill(const void* A, int dtype, int64_t lda, int64_t m,
                            int64_t n, int64_t block_size, const uint8_t* keep,
                            const int64_t* row_ptrs, int64_t n_blocks,
                            int64_t* col_indices, void* blocks, void* stream);
int tsp_bsr_to_dense(const void* blocks, int dtype, const int64_t* row_ptrs,
                     const int64_t* col_indices, int64_t n_blocks,
                     int64_t block_size, int64_t m, int64_t n, void* out,
                     int64_t ldo, void* stream);
int tsp_csr_from_dense_pattern(const void* A, int dtype, int64_t lda, int64_t m,
                               int64_t n, double threshold, int64_t* row_ptrs,
                               void* workspace, void* stream);
int tsp_csr_from_dense_fill(const void* A, int dtype, int64_t lda, int64_t m,
                            int64_t n, double threshold, const int64_t* row_ptrs,
                            int64_t* col_indices, void* values, void* stream);
int tsp_csr_to_dense(const void* values, int dtype, const int64_t* col_indices,
                     const int64_t* row_ptrs, int64_t m, int64_t n, void* out,
                     int64_t ldo, void* stream);
int tsp_csr_row_indices(const int64_t* row_ptrs, int64_t m, int64_t nnz,
                        int64_t* rows, void* stream);
int64_t tsp_coo_to_csr_workspace_size(int64_t nnz, int64_t m, int64_t n);
/* tsp_coo_sum_to_csr: as tsp_coo_to_csr, but one entry per distinct
 * (row, col) holding the sum of its duplicates in input order (explicit
 * zeros kept) — the coalesce of sparse_add (trnsparse/ops.py:107-132).
 * col_out / values_out have room for nnz entries; row_ptrs[m] is the
 * number written. workspace: tsp_coo_sum_to_csr_workspace_size bytes. */
int64_t tsp_coo_sum_to_csr_workspace_size(int64_t nnz, int64_t m, int64_t n);
int tsp_coo_sum_to_csr(const void* values, int dtype, const int64_t* row_indices,
                       const int64_t* col_indices, int64_t nnz, int64_t m,
                       int64_t n, int64_t* row_ptrs, int64_t* col_out,
                       void* values_out, void* workspace,
                       int64_t workspace_bytes, void* stream);
int tsp_coo_to_csr(const void* values, int dtype, const int64_t* row_indices,
                   const int64_t* col_indices, int64_t nnz, int64_t m,
                   int64_t n, int64_t* row_ptrs, int64_t* col_out,
                   void* values_out, void* workspace, int64_t workspace_bytes,
                   void* stream);

/* tsp_csr_transpose: CSR of A^T for A (m, n) in CSR — sparse_transpose
 * (trnsparse/ops.py:145-154: COO swap + to_csr). The entries are stably
 * sorted by column, so rows ascend within each output row and duplicates
 * keep their input order: the reference's structure and values, bit for
 * bit. out_row_ptrs (n+1,) int64, out_col / out_values (nnz,) (out_col
 * int64 = the original rows). m, n <= 2^32, nnz < 2^32. workspace:
 * tsp_csr_transpose_workspace_size(nnz, m, n, dtype) bytes. */
int64_t tsp_csr_transpose_workspace_size(int64_t nnz, int64_t m, int64_t n,
                                         int dtype);
/* tsp_csr_sum: the union sum of two CSR operands of shape (m, n) — the
 * coalesce of sparse_add (trnsparse/ops.py:107-132) with the scaled values
 * alpha*A.values / beta*B.values passed in (the caller scales them as torch
 * does). One entry per distinct (row, col), sorted by (row, col), holding
 * the sum of its duplicates in input order (A's entries before B's);
 * explicit zeros kept. col_out / values_out have room for nnz_a + nnz_b
 * entries; row_ptrs[m] is the number written. m, n, nnz_a + nnz_b <= 2^32.
 * workspace: tsp_csr_sum_workspace_size bytes. */
int64_t tsp_csr_sum_workspace_size(int64_t nnz_a, int64_t nnz_b, int64_t m,
                                   int64_t n, int dtype);
int tsp_csr_sum(const void* a_values, const int64_t* a_cols,
                const int64_t* a_row_ptrs, int64_t nnz_a, const void* b_values,
                const int64_t* b_cols, const int64_t* b_row_ptrs, int64_t nnz_b,
                int dtype, int64_t m, int64_t n, int64_t* row_ptrs,
                int64_t* col_out, void* values_out, void* workspace,
                int64_t workspace_bytes, void* stream);
int tsp_csr_transpose(const void* values, int dtype, const int64_t* col_indices,
                      const int64_t* row_ptrs, int64_t m, int64_t n,
                      int64_t nnz, int64_t* out_row_ptrs, int64_t* out_col,
                      void* out_values, void* workspace,
                      int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* TRNSPARSE_HIP_H */
