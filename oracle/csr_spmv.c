/*
 * CSR SpMV in plain C — oracle (test infrastructure only).
 *
 * Restates the reference's spmv (trnsparse/ops.py:30-48):
 *   out[i] = alpha * sum_{p in row_ptrs[i]..row_ptrs[i+1]} values[p] * x[col[p]]
 *            (+ beta * y[i] when y != NULL and beta != 0)
 * alpha applies after the row sum, y is only read, never written.
 *
 * Two variants:
 *   oracle_csr_spmv_f64  accumulates in double (parity truth, and
 *                        |A|.|x| error scale when `absolute` != 0)
 *   oracle_csr_spmv_f32  float accumulation with OpenMP over rows, the
 *                        arithmetic of the reference's fp32 path (timed as
 *                        the SpMV CPU baseline).
 * Index width is 64-bit or 32-bit (idx64 flag).
 */
#include <math.h>
#include <stdint.h>

static inline int64_t ld_idx(const void* p, int64_t i, int idx64) {
  return idx64 ? ((const int64_t*)p)[i] : (int64_t)((const int32_t*)p)[i];
}

void oracle_csr_spmv_f64(const float* values, const void* col, const void* row_ptrs, int idx64, int64_t m,
                         const float* x, double alpha, const float* y, double beta, int absolute, double* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < m; ++i) {
    double s = 0.0;
    const int64_t e = ld_idx(row_ptrs, i + 1, idx64);
    for (int64_t p = ld_idx(row_ptrs, i, idx64); p < e; ++p) {
      double v = values[p], xv = x[ld_idx(col, p, idx64)];
      s += absolute ? fabs(v) * fabs(xv) : v * xv;
    }
    s *= absolute ? fabs(alpha) : alpha;
    if (y && beta != 0.0) s += absolute ? fabs(beta) * fabs((double)y[i]) : beta * (double)y[i];
    out[i] = s;
  }
}

void oracle_csr_spmv_f32(const float* values, const void* col, const void* row_ptrs, int idx64, int64_t m,
                         const float* x, float alpha, const float* y, float beta, float* out) {
#pragma omp parallel for schedule(static, 4096)
  for (int64_t i = 0; i < m; ++i) {
    float s = 0.0f;
    const int64_t e = ld_idx(row_ptrs, i + 1, idx64);
    for (int64_t p = ld_idx(row_ptrs, i, idx64); p < e; ++p) s += values[p] * x[ld_idx(col, p, idx64)];
    float r = alpha * s;
    if (y && beta != 0.0f) r = r + beta * y[i];
    out[i] = r;
  }
}
