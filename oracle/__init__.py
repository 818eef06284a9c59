"""CPU oracle for the NF4 frozen-weight path.

TEST INFRASTRUCTURE ONLY. This package restates, on the CPU, the arithmetic
that h4rm0n1c/stratum delegates to ``bitsandbytes.functional`` on its NF4 path
(``stratum/upload.py:367-369,725-727`` quantize, ``stratum/upload.py:221,946,1038``
and ``stratum/nf4_linear.py:46`` dequantize). Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the checker. The product (``stratum_amd``) never imports,
links or calls anything here.

Pinning status per function (what checks it besides its own formula):

* ``NF4_CODE``          -- recomputed from the QLoRA normal-quantile construction
                          with scipy, sorted/endpoint invariants.
* ``block_absmax``      -- brute-force per-block max on small inputs, NaN/zero cases.
* ``nf4_codes``         -- float64 brute-force nearest level away from midpoints,
                          special values, exhaustive fp32 boundary search, and the
                          C restatement (different formulation: literal 16-way
                          argmin and a literal comparison tree).
* ``pack_nibbles``      -- known-answer byte vectors, odd-length padding.
* ``dequantize``        -- torch's own fp32->fp16/bf16 conversion on the same
                          products; endpoint values (code 0/7/15).
* Near-midpoint tie behaviour of the *installed* bitsandbytes build is
  **parity unpinned**: bitsandbytes is not importable here and its version is
  not pinned by the reference (``pyproject.toml:19``). Both of its published
  rounding rules are implemented ("argmin" = torch/CPU backend,
  "threshold" = CUDA kernel) and their disagreements are counted.
"""
