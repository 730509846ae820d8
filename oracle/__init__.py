"""CPU oracle for grout's attention hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package; the product (``grout_amd``) never does.  The C
restatement lives in ``grout_oracle.c`` (each function cites the reference
file:line it follows) and is built by ``oracle/Makefile`` into
``oracle/_build/libgrout_oracle.so``.

Parity pinning (what checks each function independently of its own formula):

* ``fill_normal_f16`` / ``fill_uniform_f16``: committed first-8-values
  self-test vectors, moments of a large sample, and an f64 -> f16 rounding
  check against numpy's own ``float64 -> float16`` cast.
* ``f2h`` / ``h2f``: exhaustive round trip over all 65536 half patterns and
  agreement with numpy's float32 -> float16 cast on random and tie inputs.
* ``rope_table``: numpy float64 recomputation, cos^2+sin^2=1, position 0 is the
  identity; ``rope_rows``: equal to the table's rows, and numpy float64 at the
  last rows of a 2^22-position cache.
* ``qk_norm_rope_row``: torch ``rms_norm`` + complex-multiplication RoPE in
  float64 (within f16 rounding), RMSNorm scale invariance, RoPE norm
  preservation and relative-position property.
* ``attention_prefill_rows`` / ``attention_decode``: torch float64
  ``scaled_dot_product_attention`` with GQA (a library implementation),
  brute-force float64 softmax on tiny shapes, closed forms (V constant,
  K constant, ctx=1, q = lambda*k_j), GQA == MHA with repeated K/V; the
  benchmark configurations against committed torch float64 fixtures
  (tests/golden/).
* ``decode_split`` + ``splitk_merge``: equal to ``attention_decode`` for every
  split count, including empty splits.
"""
from .oracle import *  # noqa: F401,F403
