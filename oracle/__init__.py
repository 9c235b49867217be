"""CPU oracle for the saeflow SAE hot path — TEST INFRASTRUCTURE, NOT PRODUCT CODE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package, and only as the checker (or, in bench.py, as the timed CPU baseline). The product
(saeflow_amd) never imports it and has no CPU path.

Modules (each function cites the reference file:line it restates):
  reference  plain-PyTorch SAE math on CPU (saeflow/reference.py:36-52, ops.py:12-49)
  csr        bit-level dense<->CSR, the CSR gather decode, row top-k (numpy)
             (saeflow/kernels/decode.py:28-126, ops.py:12-36)
  brute      pure-Python loop versions for tiny inputs: the independent pins of the two
             modules above (closed forms evaluated element by element in float64)
  backward   float64 autograd of the forward above on a given nonzero set (the gradients
             the backward kernels must give; pinned by finite differences)

Pinning (tests/test_oracle.py): every function is checked against brute force on tiny
inputs, against a library routine where one exists (torch.Tensor.to_sparse_csr,
torch.topk, a dense matmul), against the committed golden fixtures in tests/golden/, and
against known answers (all-zero input, empty rows); planted mistakes (sign of b_dec,
transposed weights, dropped bias, shifted indptr, reversed tie order) are shown to fail
those checks. The reference's own tests hold no golden vectors (all differential), so the
fixtures are written by tests/golden/make_golden.py from the brute-force pins.
"""
