"""CPU oracle for the FlashFFN v3 hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the algorithm of the reference's FlashFFN v3
path (SDMuhsin/CompAct `src/flashffn.py:995-2230`) so that the HIP kernels in
`compact_amd` can be checked against it.  It is the checker, never the thing
measured or shipped: only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` may import it.  The product (`compact_amd`)
never imports it and raises when its HIP library is missing.

Modules
  codec.py        numpy restatement of the per-group absmax codec (a1/a2), the
                  GLU elementwise math (a5), K1/K2 contracts (a3/a4) and the
                  outlier-channel extension; every function cites the
                  reference line it follows.
  exact.py        exact-rational (fractions.Fraction) brute force of the codec
                  for tiny inputs: an independent implementation that pins the
                  IEEE rounding steps of codec.py.
  codec_ref.c     plain-C restatement of the codec with its own bit-level
                  fp16/bf16 rounding, built by oracle/Makefile into
                  oracle/_build/liboracle_codec.so and bound by c_codec.py.
  flashffn_ref.py torch-CPU restatement of FlashFFNv3Function /
                  FlashFFNv3AdapterFunction forward+backward in the reference op
                  order, the fp32 plain-autograd reference of the same factored
                  computation, and the saved-bytes accounting.

Parity status per function is stated in each module header.
"""
