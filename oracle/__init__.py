"""CPU oracle for the fused dequantize+GEMM path. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import,
link or run anything in this directory, and only as the checker (or, for the
baseline, as the timed CPU comparison). The product (lowbit_amd) never imports
it: its GEMMs run on the GPU or fail loudly.

Contents
  reference.py   numpy restatement of the reference's ground truth: nibble
                 unpacking, int4/MXFP4 dequantization, float64 GEMMs, exact
                 int64 W4A8 group accumulators, the per-token int8 quantizer.
  csrc/          plain-C restatement of the same (the bit-exact quantizer, the
                 int64 group accumulators, float64 GEMMs), built into
                 oracle/_build/liblowbit_oracle.so; it checks the GPU at sizes
                 where numpy's int64 einsum is too slow.
  cref.py        ctypes loaders for that library and for oracle/_ref.
  Makefile       builds oracle/_build (own sources) and, where the reference
                 tree is mounted, oracle/_ref/liblowbit_ref.so from the
                 reference's own C sources, unmodified, in place.

Parity pinning (what checks each oracle function; see tests/test_oracle.py):
  unpack / dequantize      reference KATs for the nibble layout, the E2M1 table
                           and E8M0 decode (tests/test_formats.py of the
                           reference); round trips against independent packers
  act quantizer            bit-exact against oracle/_ref's lb_quant_act_int8
                           (the reference C), including a .5 tie and zero rows
  int64 group accumulators bit-exact against oracle/_ref's lb_w4a8_group_acc
                           (scalar and VNNI), the worst-case fixture, and brute
                           force loops on tiny inputs
  float64 GEMMs            brute-force loops on tiny inputs, closed forms (a
                           constant code row gives s*(q-z)*sum(x)), and the
                           reference C GEMMs within the 1e-5 |X||W|^T bound
"""
