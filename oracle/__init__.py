"""CPU oracle for the EPTQ quantized-Linear path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU with numpy (and torch CPU for the timed
baseline), the reference algorithms the HIP path must reproduce:

* ``codebooks``  — the reference's own table procedures: the E8-D4 heap walk
  (``quantizers/e8_d4.py:40-86``), the E8 shell expansion with lexicographic
  row deduplication (``quantizers/e8_lattice.py:54-81``) and ``remove_last``
  (``quantize.py:178-181``), the radius scaling (``reconstruct.py:52-62``,
  ``quantizers/e8_d4.py:90-102``).
* ``dequant``    — ``dequantize_layer`` (``algorithms/eptq.py:406-471``), the
  bit-exact definition of the fp16 weight, plus the CSR build of
  ``kernels/linear.py:122-139``.
* ``matvec``     — the fused decode math of ``test_e8_cuda.py:23-53`` /
  ``csrc/eptq_kernels.cu:161-292`` in float64, and the reference's CPU path
  (dequantize + fp32 matmul).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package, and only as the checker or the
timed CPU baseline — never as the thing measured on the GPU or shipped.

Pinning (what checks each function against something other than itself):

* codebooks: the heap walk and the shell expansion are compared with the
  package's closed-form enumerations (two independent constructions), with the
  theta-series shell sizes 240·σ₃(k), coset sizes, distinctness and the
  reserved (3,127,127) slot.
* dequant: known answers (g = h = 1 and no S ⇒ W = fp16(table); an index sweep
  that dumps every table row through the decode; critical-block overwrite
  order), brute-force scalar evaluation on tiny layers, and fp16 subnormal
  rounding checked against numpy's IEEE conversion.
* matvec: linearity in x, x = 0 ⇒ y = bias, g-scaling, and agreement with a
  float64 dense product of the oracle's own W.

Parity unpinned: the reference built its E8 table on whatever device
quantization ran on; checkpoints carry ``raw_codes`` so the loaded table is
the file's, but the synthetic E8 table here is pinned only by CPU ordering
rules (``torch.unique(dim=0)`` sorts rows lexicographically), not by a
reference-produced golden file (none exists in the reference).
"""
