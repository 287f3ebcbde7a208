"""CPU oracle for Kshipra's weight-only quantized linear path.

TEST INFRASTRUCTURE ONLY.  This package restates the reference algorithm
(Kshipra ``engine/quantization.py`` and the decoder op order of
``engine/model.py``) on the CPU so that the HIP kernels can be checked
against it.  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import it, and there only as the checker or as the
timed CPU baseline; ``kshipra_amd`` never imports it and has no CPU fallback.

Contents
--------
``quant``    quantize / pack / dequantize / linear, twice: a C restatement
             (``kq_oracle.c``, loaded with ctypes) and an independent numpy
             restatement.  Both follow ``engine/quantization.py:180-396``.
``decoder``  a numpy fp32 decoder step (RMSNorm, q/k/v, RoPE, causal GQA
             attention, o, SiLU-gated MLP, final norm, lm_head, argmax) in the
             op order of ``engine/model.py:93-205``, used for greedy-token parity.
``attention`` the paged K/V store (``engine/model.py:124-129``), the chunked
             online-softmax attention (``engine/chunked_prefill.py:93-140``)
             and the monolithic masked softmax (``:47-90``), float64.

How the oracle is pinned (each check is in ``tests/test_oracle_*.py``):

* exact-rational restatement (Python ``fractions``) on adversarial inputs:
  ties at .5, subnormal and underflowing scales, zero rows, tiny rows whose
  fp16 scale is 0 (the +-inf -> clamp case), large magnitudes;
* the reference tests' own known answers (``tests/test_quantization.py``):
  the 1x1 weight, the all-zero row, storage bytes, bits per weight, padding;
* invariants the reference states: the half-scale error bound, the q ranges,
  the max element mapping to +-127, sign symmetry;
* brute force over all 256 packed bytes for unpack / sign restore;
* the fp32 -> fp16 conversion against numpy's independent implementation over
  every fp16 boundary and tie;
* C restatement == numpy restatement on seeded random weights;
* attention: chunked == monolithic on the reference tests' configurations
  (its own golden relation) and closed forms (single key, equal keys, a
  dominant key, the GQA head map, the causal mask).
"""
