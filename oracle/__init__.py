"""CPU oracle of the trnsparse compute path — test infrastructure only.

Imported by `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of
`bench.py`, as the checker / the reported CPU baseline; never by the
product package `trnsparse_amd`.

Modules
- ref.py          numpy float64 restatement of the reference semantics
                  (parity truth; each function cites the reference file:line).
- cpu_baseline.py the reference's own torch path restated op for op on CPU
                  tensors (timed as the CPU baseline).
- csr_spmv.c      plain-C CSR SpMV (OpenMP), an independent implementation
                  for full-size SpMV parity and the SpMV CPU baseline.

The reference (trnsci/trnsparse) is pure Python: there is no C/C++ source to
compile into oracle/_ref, so every function here is a restatement.
"""
