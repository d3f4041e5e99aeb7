// PyTorch operator library over the C ABI: torch.ops.trnsparse_hip.*
//
// The reference reaches its device kernels through Python-level dispatch
// (trnsparse/ops.py:67-73, 204-209, 255-260, 500-505, 535-540 call into
// trnsparse/nki/dispatch.py). Here the same seam is a set of registered
// operators, so the kernels are visible to the dispatcher: torch.compile
// traces them through their Meta implementations (shapes and dtypes only),
// they run on the current HIP stream (graph capture records them like any
// other op), and C++ callers can use them without Python.
//
// Each operator allocates its outputs (and any workspace) with torch, takes
// device pointers and strides from contiguous tensors, calls one entry point
// of libtrnsparse_hip.so and turns a non-zero status into an exception
// carrying tsp_last_error(). The Python layer (trnsparse_amd/hip/dispatch.py)
// keeps the planning and caching (row orders, CSR windows and column plans,
// the attention backward's column plan) and the autograd wrappers.
#include <ATen/ATen.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <algorithm>
#include <string>
#include <tuple>

#include "trnsparse_hip.h"

namespace {

void check(int status, const char* who) {
  TORCH_CHECK(status == TSP_OK, who, " failed with status ", status, ": ", tsp_last_error());
}

void* stream_of(const at::Tensor& t) {
  return (void*)c10::hip::getCurrentHIPStream(t.device().index()).stream();
}

int dtype_code(at::ScalarType t) {
  switch (t) {
    case at::kFloat: return TSP_F32;
    case at::kDouble: return TSP_F64;
    case at::kBFloat16: return TSP_BF16;
    default: TORCH_CHECK(false, "trnsparse_hip: dtype ", t, " not supported");
  }
  return -1;
}

int index_code(at::ScalarType t) {
  TORCH_CHECK(t == at::kInt || t == at::kLong, "trnsparse_hip: index dtype ", t, " not supported");
  return t == at::kInt ? TSP_I32 : TSP_I64;
}

// a tensor the kernels may read: on `dev`, contiguous
void need(const at::Tensor& t, const at::Tensor& like, const char* name) {
  TORCH_CHECK(t.device() == like.device(), "trnsparse_hip: ", name, " is on ", t.device(), ", expected ",
              like.device());
  TORCH_CHECK(t.is_contiguous(), "trnsparse_hip: ", name, " must be contiguous");
}

const void* opt_ptr(const c10::optional<at::Tensor>& t) { return t.has_value() ? t->data_ptr() : nullptr; }

// The operators are public (C++ callers and torch.ops users reach them
// without the Python layer), and the kernels trust every size they are
// given: each operator checks that its tensors match the sizes, dtypes and
// index widths it passes on, so a mismatched call raises here instead of
// launching a kernel that reads or writes past a buffer.
void need_dtype(const at::Tensor& t, at::ScalarType dt, const char* op, const char* name) {
  TORCH_CHECK(t.scalar_type() == dt, op, ": ", name, " has dtype ", t.scalar_type(), ", expected ", dt);
}

void need_numel(const at::Tensor& t, int64_t n, const char* op, const char* name) {
  TORCH_CHECK(t.numel() == n, op, ": ", name, " has ", t.numel(), " elements, expected ", n);
}

void need_2d(const at::Tensor& t, int64_t rows, int64_t cols, const char* op, const char* name) {
  TORCH_CHECK(t.dim() == 2 && t.size(0) == rows && t.size(1) == cols, op, ": ", name, " has shape ", t.sizes(),
              ", expected [", rows, ", ", cols, "]");
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// A BSR pattern of an m x n matrix in b x b blocks: int64 row pointers over
// the block rows, int64 column indices and (nnzb, b, b) blocks.
void need_bsr(const at::Tensor& blocks, const at::Tensor& rp, const at::Tensor& ci, int64_t m, int64_t n,
              int64_t b, const char* op) {
  TORCH_CHECK(m >= 0 && n >= 0 && b > 0, op, ": bad sizes m=", m, " n=", n, " block_size=", b);
  need_dtype(rp, at::kLong, op, "block_row_ptrs");
  need_dtype(ci, at::kLong, op, "block_col_indices");
  need_numel(rp, cdiv(m, b) + 1, op, "block_row_ptrs");
  TORCH_CHECK(blocks.dim() == 3 && blocks.size(1) == b && blocks.size(2) == b, op, ": blocks has shape ",
              blocks.sizes(), ", expected [nnzb, ", b, ", ", b, "]");
  need_numel(ci, blocks.size(0), op, "block_col_indices");
}

// ------------------------------------------------------------------- BSR

at::Tensor bsr_spmm(const at::Tensor& blocks, const at::Tensor& rp, const at::Tensor& ci,
                    const c10::optional<at::Tensor>& row_order, int64_t m, int64_t n, int64_t block_size,
                    const at::Tensor& B, at::ScalarType out_dtype) {
  for (auto* p : {&rp, &ci}) need(*p, B, "pattern");
  need(blocks, B, "blocks");
  TORCH_CHECK(B.dim() == 2 && B.stride(1) == 1, "bsr_spmm: B must be 2-D with unit column stride");
  need_bsr(blocks, rp, ci, m, n, block_size, "bsr_spmm");
  need_dtype(blocks, B.scalar_type(), "bsr_spmm", "blocks (the dtype of B)");
  TORCH_CHECK(B.size(0) >= n, "bsr_spmm: B has ", B.size(0), " rows, expected at least n = ", n);
  TORCH_CHECK(B.stride(0) >= B.size(1), "bsr_spmm: B's row stride ", B.stride(0), " is below its ", B.size(1),
              " columns");
  if (row_order.has_value() && row_order->numel()) {
    need(*row_order, B, "row_order");
    need_dtype(*row_order, at::kInt, "bsr_spmm", "row_order");
    TORCH_CHECK(row_order->numel() >= cdiv(m, block_size), "bsr_spmm: row_order has ", row_order->numel(),
                " entries for ", cdiv(m, block_size), " block rows");
  }
  const int64_t ncols = B.size(1);
  auto C = at::empty({m, ncols}, B.options().dtype(out_dtype));
  const int32_t* order = row_order.has_value() && row_order->numel() ? row_order->data_ptr<int32_t>() : nullptr;
  check(tsp_bsr_spmm(blocks.data_ptr(), dtype_code(blocks.scalar_type()), rp.data_ptr<int64_t>(),
                     ci.data_ptr<int64_t>(), blocks.size(0), block_size, m, n, B.data_ptr(), B.stride(0), ncols,
                     C.data_ptr(), ncols, dtype_code(out_dtype), order, stream_of(B)),
        "tsp_bsr_spmm");
  return C;
}

at::Tensor bsr_spmm_meta(const at::Tensor& blocks, const at::Tensor&, const at::Tensor&,
                         const c10::optional<at::Tensor>&, int64_t m, int64_t, int64_t, const at::Tensor& B,
                         at::ScalarType out_dtype) {
  return at::empty({m, B.size(1)}, B.options().dtype(out_dtype));
}

at::Tensor bsr_sddmm(const at::Tensor& G, const at::Tensor& B, const at::Tensor& block_rows,
                     const at::Tensor& block_col_indices, int64_t m, int64_t n, int64_t block_size) {
  need(G, G, "dC");
  need(B, G, "B");
  need(block_rows, G, "block_rows");
  need(block_col_indices, G, "block_col_indices");
  TORCH_CHECK(m >= 0 && n >= 0 && block_size > 0, "bsr_sddmm: bad sizes");
  TORCH_CHECK(G.dim() == 2 && G.size(0) == m, "bsr_sddmm: grad_out has shape ", G.sizes(), ", expected [", m,
              ", N]");
  need_2d(B, n, G.size(1), "bsr_sddmm", "B");
  need_dtype(B, G.scalar_type(), "bsr_sddmm", "B (the dtype of grad_out)");
  need_dtype(block_rows, at::kLong, "bsr_sddmm", "block_rows");
  need_dtype(block_col_indices, at::kLong, "bsr_sddmm", "block_col_indices");
  need_numel(block_rows, block_col_indices.numel(), "bsr_sddmm", "block_rows");
  const int64_t nnzb = block_col_indices.numel(), ncols = G.size(1);
  auto out = at::empty({nnzb, block_size, block_size}, G.options());
  check(tsp_bsr_sddmm(G.data_ptr(), ncols, m, B.data_ptr(), ncols, n, ncols, block_rows.data_ptr<int64_t>(),
                      block_col_indices.data_ptr<int64_t>(), nnzb, block_size, dtype_code(G.scalar_type()),
                      out.data_ptr(), stream_of(G)),
        "tsp_bsr_sddmm");
  return out;
}

at::Tensor bsr_sddmm_meta(const at::Tensor& G, const at::Tensor&, const at::Tensor&,
                          const at::Tensor& block_col_indices, int64_t, int64_t, int64_t block_size) {
  return at::empty({block_col_indices.size(0), block_size, block_size}, G.options());
}

at::Tensor bsr_spmm_t(const at::Tensor& blocks, const at::Tensor& cp, const at::Tensor& cbid, const at::Tensor& crow,
                      const at::Tensor& col_order, int64_t m, int64_t n, int64_t block_size, const at::Tensor& G) {
  for (auto* p : {&blocks, &cp, &cbid, &crow, &col_order}) need(*p, G, "pattern");
  need(G, G, "dC");
  TORCH_CHECK(m >= 0 && n >= 0 && block_size > 0, "bsr_spmm_t: bad sizes");
  TORCH_CHECK(G.dim() == 2 && G.size(0) == m, "bsr_spmm_t: grad_out has shape ", G.sizes(), ", expected [", m,
              ", N]");
  TORCH_CHECK(blocks.dim() == 3 && blocks.size(1) == block_size && blocks.size(2) == block_size,
              "bsr_spmm_t: blocks has shape ", blocks.sizes());
  need_dtype(blocks, G.scalar_type(), "bsr_spmm_t", "blocks (the dtype of grad_out)");
  for (auto* p : {&cp, &cbid, &crow}) need_dtype(*p, at::kLong, "bsr_spmm_t", "column view");
  need_numel(cp, cdiv(n, block_size) + 1, "bsr_spmm_t", "col_ptrs");
  need_numel(cbid, blocks.size(0), "bsr_spmm_t", "col_block_ids");
  need_numel(crow, blocks.size(0), "bsr_spmm_t", "col_block_rows");
  if (col_order.numel()) {
    need_dtype(col_order, at::kInt, "bsr_spmm_t", "col_order");
    TORCH_CHECK(col_order.numel() >= cdiv(n, block_size), "bsr_spmm_t: col_order has ", col_order.numel(),
                " entries for ", cdiv(n, block_size), " block columns");
  }
  const int64_t ncols = G.size(1), nbc = cp.numel() - 1;
  auto out = at::empty({n, ncols}, G.options());
  check(tsp_bsr_spmm_t(blocks.data_ptr(), dtype_code(blocks.scalar_type()), cp.data_ptr<int64_t>(),
                       cbid.data_ptr<int64_t>(), crow.data_ptr<int64_t>(), nbc, block_size, m, n, G.data_ptr(), ncols,
                       ncols, out.data_ptr(), ncols, col_order.numel() ? col_order.data_ptr<int32_t>() : nullptr,
                       stream_of(G)),
        "tsp_bsr_spmm_t");
  return out;
}

at::Tensor bsr_spmm_t_meta(const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&,
                           const at::Tensor&, int64_t, int64_t n, int64_t, const at::Tensor& G) {
  return at::empty({n, G.size(1)}, G.options());
}

// ------------------------------------------------------------------- CSR

// A CSR matrix of m rows and n columns whose values share the dense
// operand's dtype, with one index dtype for both index arrays.
void need_csr(const at::Tensor& values, const at::Tensor& cols, const at::Tensor& ptrs, int64_t m, int64_t n,
              const at::Tensor& dense, const char* op) {
  TORCH_CHECK(m >= 0 && n >= 0, op, ": bad sizes m=", m, " n=", n);
  need_dtype(values, dense.scalar_type(), op, "values (the dtype of the dense operand)");
  index_code(cols.scalar_type());
  need_dtype(ptrs, cols.scalar_type(), op, "row_ptrs (the dtype of col_indices)");
  need_numel(ptrs, m + 1, op, "row_ptrs");
  need_numel(cols, values.numel(), op, "col_indices");
}

at::Tensor csr_spmv(const at::Tensor& values, const at::Tensor& cols, const at::Tensor& ptrs,
                    const at::Tensor& windows, int64_t m, int64_t n, const at::Tensor& x, double alpha,
                    const c10::optional<at::Tensor>& y, double beta) {
  for (auto* p : {&values, &cols, &ptrs, &windows}) need(*p, x, "matrix");
  need(x, x, "x");
  if (y.has_value()) need(*y, x, "y");
  need_csr(values, cols, ptrs, m, n, x, "csr_spmv");
  need_numel(x, n, "csr_spmv", "x");
  if (y.has_value()) {
    need_dtype(*y, x.scalar_type(), "csr_spmv", "y (the dtype of x)");
    need_numel(*y, m, "csr_spmv", "y");
  }
  need_dtype(windows, at::kLong, "csr_spmv", "windows");
  TORCH_CHECK(windows.numel() >= tsp_csr_plan_size(m, values.numel()), "csr_spmv: windows has ", windows.numel(),
              " entries, tsp_csr_plan_size gives ", tsp_csr_plan_size(m, values.numel()));
  auto out = at::empty({m}, x.options());
  check(tsp_csr_spmv(values.data_ptr(), dtype_code(values.scalar_type()), cols.data_ptr(), ptrs.data_ptr(),
                     index_code(cols.scalar_type()), m, n, values.numel(), windows.data_ptr<int64_t>(), x.data_ptr(),
                     alpha, opt_ptr(y), beta, out.data_ptr(), stream_of(x)),
        "tsp_csr_spmv");
  return out;
}

at::Tensor csr_spmv_meta(const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&, int64_t m,
                         int64_t, const at::Tensor& x, double, const c10::optional<at::Tensor>&, double) {
  return at::empty({m}, x.options());
}

// The geometry is the 10 host values of tsp_csr_colplan_geometry as an int
// list (not a tensor: a CPU tensor beside device tensors cannot be traced
// by torch.compile's fake tensors).
at::Tensor csr_colplan_spmv(const at::Tensor& plan, at::IntArrayRef geometry, const at::Tensor& values,
                            const at::Tensor& cols, const at::Tensor& ptrs, int64_t m, int64_t n, const at::Tensor& x,
                            double alpha, const c10::optional<at::Tensor>& y, double beta) {
  need(plan, x, "plan");
  for (auto* p : {&values, &cols, &ptrs}) need(*p, x, "matrix");
  need(x, x, "x");
  if (y.has_value()) need(*y, x, "y");
  TORCH_CHECK(geometry.size() == 10,
              "csr_colplan_spmv: geometry must be the 10 int64 host values of tsp_csr_colplan_geometry");
  const int64_t* geom = geometry.data();
  need_csr(values, cols, ptrs, m, n, x, "csr_colplan_spmv");
  need_dtype(x, at::kFloat, "csr_colplan_spmv", "x");
  need_numel(x, n, "csr_colplan_spmv", "x");
  if (y.has_value()) {
    need_dtype(*y, at::kFloat, "csr_colplan_spmv", "y");
    need_numel(*y, m, "csr_colplan_spmv", "y");
  }
  TORCH_CHECK(plan.nbytes() >= (size_t)geom[6], "csr_colplan_spmv: plan holds ", plan.nbytes(),
              " bytes, the geometry needs ", geom[6]);
  auto out = at::empty({m}, x.options());
  at::Tensor work = at::empty({geom[8]}, x.options().dtype(at::kByte));
  check(tsp_csr_colplan_spmv(plan.data_ptr(), dtype_code(x.scalar_type()), m, n, values.numel(), geom,
                             values.data_ptr(), cols.data_ptr(), ptrs.data_ptr(), index_code(cols.scalar_type()),
                             x.data_ptr(), alpha, opt_ptr(y), beta, out.data_ptr(), work.data_ptr(), stream_of(x)),
        "tsp_csr_colplan_spmv");
  return out;
}

at::Tensor csr_colplan_spmv_meta(const at::Tensor&, at::IntArrayRef, const at::Tensor&, const at::Tensor&,
                                 const at::Tensor&, int64_t m, int64_t, const at::Tensor& x, double,
                                 const c10::optional<at::Tensor>&, double) {
  return at::empty({m}, x.options());
}

at::Tensor csr_spmm(const at::Tensor& values, const at::Tensor& cols, const at::Tensor& ptrs, int64_t m, int64_t n,
                    const at::Tensor& X, double alpha, const c10::optional<at::Tensor>& Y, double beta) {
  for (auto* p : {&values, &cols, &ptrs}) need(*p, X, "matrix");
  need(X, X, "X");
  if (Y.has_value()) need(*Y, X, "Y");
  need_csr(values, cols, ptrs, m, n, X, "csr_spmm");
  TORCH_CHECK(X.dim() == 2 && X.size(0) == n, "csr_spmm: X has shape ", X.sizes(), ", expected [", n, ", N]");
  const int64_t ncols = X.size(1);
  if (Y.has_value()) {
    need_dtype(*Y, X.scalar_type(), "csr_spmm", "Y (the dtype of X)");
    need_2d(*Y, m, ncols, "csr_spmm", "Y");
  }
  auto out = at::empty({m, ncols}, X.options());
  check(tsp_csr_spmm(values.data_ptr(), dtype_code(values.scalar_type()), cols.data_ptr(), ptrs.data_ptr(),
                     index_code(cols.scalar_type()), m, n, values.numel(), X.data_ptr(), ncols, ncols, alpha,
                     opt_ptr(Y), ncols, beta, out.data_ptr(), ncols, stream_of(X)),
        "tsp_csr_spmm");
  return out;
}

at::Tensor csr_spmm_meta(const at::Tensor&, const at::Tensor&, const at::Tensor&, int64_t m, int64_t,
                         const at::Tensor& X, double, const c10::optional<at::Tensor>&, double) {
  return at::empty({m, X.size(1)}, X.options());
}

// -------------------------------------------------------------- screened

at::Tensor screened_workspace(const at::Tensor& diag, int64_t m) {
  const int64_t bytes = tsp_screened_workspace_size(m, dtype_code(diag.scalar_type()));
  TORCH_CHECK(bytes >= 0, "tsp_screened_workspace_size failed: ", tsp_last_error());
  return at::empty({bytes > 0 ? bytes : 1}, diag.options().dtype(at::kByte));
}

at::Tensor screened_spmm(const at::Tensor& A, const at::Tensor& diag, const at::Tensor& B, double threshold_sqrt) {
  need(A, B, "A");
  need(diag, B, "diag_integrals");
  need(B, B, "B");
  TORCH_CHECK(A.dim() == 2 && A.size(0) == A.size(1), "screened_spmm: A has shape ", A.sizes(), ", expected square");
  const int64_t m = A.size(0);
  TORCH_CHECK(B.dim() == 2 && B.size(0) == m, "screened_spmm: B has shape ", B.sizes(), ", expected [", m, ", N]");
  need_dtype(A, B.scalar_type(), "screened_spmm", "A (the dtype of B)");
  TORCH_CHECK(diag.dim() == 1, "screened_spmm: diag_integrals must be 1-D");
  need_numel(diag, m, "screened_spmm", "diag_integrals");
  const int64_t ncols = B.size(1);
  auto C = at::empty({m, ncols}, B.options());
  auto ws = screened_workspace(diag, m);
  check(tsp_screened_spmm(A.data_ptr(), dtype_code(A.scalar_type()), A.size(1), diag.data_ptr(),
                          dtype_code(diag.scalar_type()), threshold_sqrt, m, B.data_ptr(), ncols, ncols, C.data_ptr(),
                          ncols, ws.data_ptr(), stream_of(B)),
        "tsp_screened_spmm");
  return C;
}

at::Tensor screened_spmm_meta(const at::Tensor& A, const at::Tensor&, const at::Tensor& B, double) {
  return at::empty({A.size(0), B.size(1)}, B.options());
}

std::tuple<at::Tensor, at::Tensor> screened_spmm_backward(const at::Tensor& A, const at::Tensor& diag,
                                                          const at::Tensor& B, double threshold_sqrt,
                                                          const at::Tensor& dC, bool need_a, bool need_b) {
  need(A, dC, "A");
  need(diag, dC, "diag_integrals");
  need(B, dC, "B");
  need(dC, dC, "grad_out");
  TORCH_CHECK(A.dim() == 2 && A.size(0) == A.size(1), "screened_spmm_backward: A has shape ", A.sizes(),
              ", expected square");
  const int64_t m = A.size(0);
  TORCH_CHECK(dC.dim() == 2 && dC.size(0) == m, "screened_spmm_backward: grad_out has shape ", dC.sizes(),
              ", expected [", m, ", N]");
  need_2d(B, m, dC.size(1), "screened_spmm_backward", "B");
  need_dtype(A, dC.scalar_type(), "screened_spmm_backward", "A (the dtype of grad_out)");
  need_dtype(B, dC.scalar_type(), "screened_spmm_backward", "B (the dtype of grad_out)");
  TORCH_CHECK(diag.dim() == 1, "screened_spmm_backward: diag_integrals must be 1-D");
  need_numel(diag, m, "screened_spmm_backward", "diag_integrals");
  const int64_t ncols = dC.size(1);
  // a gradient that is not asked for comes back empty (no kernel runs for it)
  auto dA = need_a ? at::empty({m, m}, A.options()) : at::empty({0}, A.options());
  auto dB = need_b ? at::empty({m, ncols}, B.options()) : at::empty({0}, B.options());
  auto ws = screened_workspace(diag, m);
  check(tsp_screened_spmm_backward(A.data_ptr(), dtype_code(A.scalar_type()), m, diag.data_ptr(),
                                   dtype_code(diag.scalar_type()), threshold_sqrt, m, B.data_ptr(), ncols, ncols,
                                   dC.data_ptr(), ncols, need_a ? dA.data_ptr() : nullptr, m,
                                   need_b ? dB.data_ptr() : nullptr, ncols, ws.data_ptr(), stream_of(dC)),
        "tsp_screened_spmm_backward");
  return {dA, dB};
}

std::tuple<at::Tensor, at::Tensor> screened_spmm_backward_meta(const at::Tensor& A, const at::Tensor&,
                                                               const at::Tensor& B, double, const at::Tensor& dC,
                                                               bool need_a, bool need_b) {
  const int64_t m = A.size(0);
  return {need_a ? at::empty({m, m}, A.options()) : at::empty({0}, A.options()),
          need_b ? at::empty({m, dC.size(1)}, B.options()) : at::empty({0}, B.options())};
}

// ------------------------------------------------------------- attention

at::ScalarType stat_dtype(const at::Tensor& Q) { return Q.scalar_type() == at::kDouble ? at::kDouble : at::kFloat; }

std::tuple<at::Tensor, at::Tensor, at::Tensor> bsa_fwd(const at::Tensor& Q, const at::Tensor& K, const at::Tensor& V,
                                                       const at::Tensor& rp, const at::Tensor& ci, int64_t block_size,
                                                       double scale, bool return_stats) {
  for (auto* p : {&K, &V, &rp, &ci}) need(*p, Q, "operand");
  need(Q, Q, "Q");
  TORCH_CHECK(Q.dim() == 3 && K.sizes() == Q.sizes() && V.sizes() == Q.sizes(),
              "bsa_fwd: Q, K, V must be (heads, seq, head_dim) of one shape");
  TORCH_CHECK(block_size > 0, "bsa_fwd: block_size must be positive");
  for (auto* p : {&K, &V}) need_dtype(*p, Q.scalar_type(), "bsa_fwd", "K and V (the dtype of Q)");
  const int64_t H = Q.size(0), S = Q.size(1), D = Q.size(2), Mt = S / block_size;
  need_dtype(rp, at::kLong, "bsa_fwd", "block_row_ptrs");
  need_dtype(ci, at::kLong, "bsa_fwd", "block_col_indices");
  TORCH_CHECK(rp.numel() >= Mt + 1, "bsa_fwd: block_row_ptrs has ", rp.numel(), " entries, expected at least ",
              Mt + 1);
  auto O = at::empty_like(Q);
  at::Tensor rmax, rden;
  if (return_stats) {
    rmax = at::empty({H, Mt, block_size}, Q.options().dtype(stat_dtype(Q)));
    rden = at::empty({H, Mt, block_size}, Q.options().dtype(stat_dtype(Q)));
  } else {
    rmax = at::empty({0}, Q.options().dtype(stat_dtype(Q)));
    rden = at::empty({0}, Q.options().dtype(stat_dtype(Q)));
  }
  check(tsp_bsa_fwd(Q.data_ptr(), K.data_ptr(), V.data_ptr(), dtype_code(Q.scalar_type()), H, S, D,
                    rp.data_ptr<int64_t>(), ci.data_ptr<int64_t>(), block_size, scale, O.data_ptr(),
                    return_stats ? rmax.data_ptr() : nullptr, return_stats ? rden.data_ptr() : nullptr, stream_of(Q)),
        "tsp_bsa_fwd");
  return {O, rmax, rden};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> bsa_fwd_meta(const at::Tensor& Q, const at::Tensor&, const at::Tensor&,
                                                            const at::Tensor&, const at::Tensor&, int64_t block_size,
                                                            double, bool return_stats) {
  const int64_t H = Q.size(0), Mt = Q.size(1) / block_size;
  auto so = Q.options().dtype(stat_dtype(Q));
  if (!return_stats) return {at::empty_like(Q), at::empty({0}, so), at::empty({0}, so)};
  return {at::empty_like(Q), at::empty({H, Mt, block_size}, so), at::empty({H, Mt, block_size}, so)};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> bsa_bwd(
    const at::Tensor& Q, const at::Tensor& K, const at::Tensor& V, const at::Tensor& O, const at::Tensor& dO,
    const at::Tensor& rp, const at::Tensor& ci, const at::Tensor& cp, const at::Tensor& crow, int64_t n_block_cols,
    int64_t block_size, double scale, const at::Tensor& row_max, const at::Tensor& row_denom, const at::Tensor& plan,
    int64_t n_items, int64_t n_splits, int64_t n_partials) {
  for (auto* p : {&K, &V, &O, &dO, &rp, &ci, &cp, &crow, &row_max, &row_denom, &plan}) need(*p, Q, "operand");
  need(Q, Q, "Q");
  TORCH_CHECK(Q.dim() == 3, "bsa_bwd: operands must be (heads, seq, head_dim)");
  TORCH_CHECK(block_size > 0, "bsa_bwd: block_size must be positive");
  for (auto* p : {&K, &V, &O, &dO}) {
    TORCH_CHECK(p->sizes() == Q.sizes(), "bsa_bwd: K, V, O and grad_out must have Q's shape ", Q.sizes());
    need_dtype(*p, Q.scalar_type(), "bsa_bwd", "K, V, O and grad_out (the dtype of Q)");
  }
  const int64_t H = Q.size(0), S = Q.size(1), D = Q.size(2), Mt = S / block_size;
  for (auto* p : {&rp, &ci, &cp, &crow}) need_dtype(*p, at::kLong, "bsa_bwd", "mask views");
  TORCH_CHECK(rp.numel() >= Mt + 1, "bsa_bwd: block_row_ptrs has ", rp.numel(), " entries, expected at least ",
              Mt + 1);
  TORCH_CHECK(n_block_cols >= 0, "bsa_bwd: negative n_block_cols");
  need_numel(cp, n_block_cols + 1, "bsa_bwd", "col_ptrs");
  // the column view covers the stored blocks of the block rows below Mt
  TORCH_CHECK(crow.numel() <= std::max<int64_t>(ci.numel(), 1), "bsa_bwd: col_block_rows has ", crow.numel(),
              " entries, more than the mask's ", ci.numel(), " blocks");
  for (auto* p : {&row_max, &row_denom}) {
    need_dtype(*p, stat_dtype(Q), "bsa_bwd", "row_max and row_denom");
    need_numel(*p, H * Mt * block_size, "bsa_bwd", "row_max and row_denom");
  }
  need_dtype(plan, at::kInt, "bsa_bwd", "plan");
  TORCH_CHECK(n_items >= 0 && n_splits >= 0 && n_partials >= 0, "bsa_bwd: negative plan counts");
  TORCH_CHECK(plan.numel() >= 4 + 4 * n_items + 4 * n_splits, "bsa_bwd: plan has ", plan.numel(),
              " entries, its header counts need ", 4 + 4 * n_items + 4 * n_splits);
  auto dQ = at::empty_like(Q), dK = at::empty_like(Q), dV = at::empty_like(Q);
  const int64_t wsb = tsp_bsa_bwd_workspace_size(H, S, D, n_partials);
  TORCH_CHECK(wsb >= 0, "tsp_bsa_bwd_workspace_size failed: ", tsp_last_error());
  auto ws = at::empty({wsb > 0 ? wsb : 1}, Q.options().dtype(at::kByte));
  check(tsp_bsa_bwd(Q.data_ptr(), K.data_ptr(), V.data_ptr(), O.data_ptr(), dO.data_ptr(), dtype_code(Q.scalar_type()),
                    H, S, D, rp.data_ptr<int64_t>(), ci.data_ptr<int64_t>(), cp.data_ptr<int64_t>(),
                    crow.data_ptr<int64_t>(), n_block_cols, block_size, scale, row_max.data_ptr(),
                    row_denom.data_ptr(), dQ.data_ptr(), dK.data_ptr(), dV.data_ptr(), plan.data_ptr<int32_t>(),
                    n_items, n_splits, n_partials, ws.data_ptr(), stream_of(Q)),
        "tsp_bsa_bwd");
  return {dQ, dK, dV};
}

std::tuple<at::Tensor, at::Tensor, at::Tensor> bsa_bwd_meta(
    const at::Tensor& Q, const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&,
    const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&, int64_t, int64_t, double,
    const at::Tensor&, const at::Tensor&, const at::Tensor&, int64_t, int64_t, int64_t) {
  return {at::empty_like(Q), at::empty_like(Q), at::empty_like(Q)};
}

}  // namespace

TORCH_LIBRARY(trnsparse_hip, m) {
  m.def("bsr_spmm(Tensor blocks, Tensor block_row_ptrs, Tensor block_col_indices, Tensor? row_order, int m, int n, "
        "int block_size, Tensor B, ScalarType out_dtype) -> Tensor");
  m.def("bsr_sddmm(Tensor grad_out, Tensor B, Tensor block_rows, Tensor block_col_indices, int m, int n, "
        "int block_size) -> Tensor");
  m.def("bsr_spmm_t(Tensor blocks, Tensor col_ptrs, Tensor col_block_ids, Tensor col_block_rows, Tensor col_order, "
        "int m, int n, int block_size, Tensor grad_out) -> Tensor");
  m.def("csr_spmv(Tensor values, Tensor col_indices, Tensor row_ptrs, Tensor windows, int m, int n, Tensor x, "
        "float alpha, Tensor? y, float beta) -> Tensor");
  m.def("csr_colplan_spmv(Tensor plan, int[] geometry, Tensor values, Tensor col_indices, Tensor row_ptrs, int m, "
        "int n, Tensor x, float alpha, Tensor? y, float beta) -> Tensor");
  m.def("csr_spmm(Tensor values, Tensor col_indices, Tensor row_ptrs, int m, int n, Tensor X, float alpha, "
        "Tensor? Y, float beta) -> Tensor");
  m.def("screened_spmm(Tensor A, Tensor diag_integrals, Tensor B, float threshold_sqrt) -> Tensor");
  m.def("screened_spmm_backward(Tensor A, Tensor diag_integrals, Tensor B, float threshold_sqrt, Tensor grad_out, "
        "bool need_a, bool need_b) -> (Tensor, Tensor)");
  m.def("bsa_fwd(Tensor Q, Tensor K, Tensor V, Tensor block_row_ptrs, Tensor block_col_indices, int block_size, "
        "float scale, bool return_stats) -> (Tensor, Tensor, Tensor)");
  m.def("bsa_bwd(Tensor Q, Tensor K, Tensor V, Tensor O, Tensor dO, Tensor block_row_ptrs, Tensor block_col_indices, "
        "Tensor col_ptrs, Tensor col_block_rows, int n_block_cols, int block_size, float scale, Tensor row_max, "
        "Tensor row_denom, Tensor plan, int n_items, int n_splits, int n_partials) -> (Tensor, Tensor, Tensor)");
}

// the "CUDA" dispatch key is the GPU key of PyTorch-ROCm
TORCH_LIBRARY_IMPL(trnsparse_hip, CUDA, m) {
  m.impl("bsr_spmm", &bsr_spmm);
  m.impl("bsr_sddmm", &bsr_sddmm);
  m.impl("bsr_spmm_t", &bsr_spmm_t);
  m.impl("csr_spmv", &csr_spmv);
  m.impl("csr_colplan_spmv", &csr_colplan_spmv);
  m.impl("csr_spmm", &csr_spmm);
  m.impl("screened_spmm", &screened_spmm);
  m.impl("screened_spmm_backward", &screened_spmm_backward);
  m.impl("bsa_fwd", &bsa_fwd);
  m.impl("bsa_bwd", &bsa_bwd);
}

TORCH_LIBRARY_IMPL(trnsparse_hip, Meta, m) {
  m.impl("bsr_spmm", &bsr_spmm_meta);
  m.impl("bsr_sddmm", &bsr_sddmm_meta);
  m.impl("bsr_spmm_t", &bsr_spmm_t_meta);
  m.impl("csr_spmv", &csr_spmv_meta);
  m.impl("csr_colplan_spmv", &csr_colplan_spmv_meta);
  m.impl("csr_spmm", &csr_spmm_meta);
  m.impl("screened_spmm", &screened_spmm_meta);
  m.impl("screened_spmm_backward", &screened_spmm_backward_meta);
  m.impl("bsa_fwd", &bsa_fwd_meta);
  m.impl("bsa_bwd", &bsa_bwd_meta);
}
