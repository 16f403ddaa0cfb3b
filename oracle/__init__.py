"""CPU oracle for tritonkv's quantized-KV decode attention -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the algorithm of the reference's
``quantize.py`` and ``reference.py`` (and ``l2_sweep.reference_grouped``) so
that the HIP kernels in ``tritonkv_amd`` can be checked against it.  It is the
*checker*, never the thing measured or shipped: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  ``tritonkv_amd`` never imports it and has no CPU fallback.

Modules
-------
``quant``      numpy restatement of pack/unpack/quantize/dequantize
               (reference ``quantize.py:149-246``).
``attention``  numpy fp32 decode attention, flat and grouped
               (reference ``reference.py:44-88``, ``l2_sweep.py:196-236``).
``inputs``     seeded input generators (reference ``reference.py:361-392``
               plus the Llama outlier-channel and ragged-length generators the
               benchmark configurations ask for).
``splits``     restatement of the host-side split arithmetic
               (reference ``kernels/fused_decode_attn.py:398-416``, ``:486-499``).
``c_oracle``   ctypes binding of ``tkv_oracle.c``, an independent scalar C
               restatement of the quantizer, the dequantizer and the fp32
               attention (built by ``oracle/build_oracle.sh``).

How each function is pinned (so that a plausible mistake fails a test):

* pack/unpack -- exhaustive known-answer tests over all 256 byte values and
  hand-built split-P rows, plus the reference's round-trip test.
* quantize -- golden vectors written from the reference's own
  ``quantize_groupwise`` (``tests/golden/make_golden.py``), the half-step bound,
  constant-group exactness, and agreement with the independent C restatement.
* dequantize -- closed form ``fma(c, s, z)`` checked against exact float64
  arithmetic and the C restatement.
* attention -- float64 brute force on tiny inputs, S=1 gives the V row, q=0
  gives the mean of V, grouped == flat, and the reference's published
  end-to-end rel-L2 table (``README.md:286-295``).
* splits -- closed-form integer tables.
"""
