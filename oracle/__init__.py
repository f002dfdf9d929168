"""TEST INFRASTRUCTURE - the parity oracle of the `hip` backend. Not product code.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import anything here,
and only as the checker (or, for cpu_baseline, as the reported CPU baseline). The product
(clarus_amd/) never imports it: a missing HIP library fails loudly instead of falling back.

oracle.torch_ref  restates the semantics of the reference's PyTorch backend
                  (python/clarus/ops/torch_ref.py) for the GEMM-family ops plus the few
                  non-GEMM ops the NAFNet harness needs, in fp32 math on the CPU (or any torch
                  device), each function citing the reference lines it follows.

How each function is pinned (tests/test_oracle.py): against float64 brute force on small odd
shapes (matmul sums, conv windows, space-to-depth / pixel-shuffle index maps, two-pass
LayerNorm), the reference's own known-answer tests (400*200*64*1e-4 = 512, the gate 65536,
2^-6, TLC windows), numpy.fft for the patch DFT ops, and closed forms (softmax rows sum to 1,
Gram symmetry, Parseval). The reference ships no golden-vector files, so the compositions those
checks leave open (the NAFNet model adapter's fold / wiring / residual dtypes, and combined
prologue + epilogue orders of linear, ln_mul_linear, conv3x3 and linear_per_image) are pinned by
fixtures that the reference itself wrote (tests/golden/make_golden.py): tests/test_golden.py
requires the oracle to reproduce them bit for bit.
"""
