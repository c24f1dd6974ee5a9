"""CPU oracle for the sdcguard verification hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in this package is part of the product: only the tests under
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import it,
and only to check (or time, as a reported CPU baseline) what the HIP library computes.  The
product package ``sdcguard_amd`` never imports it and has no CPU fallback.

Each function restates, in numpy (float32 arithmetic where the reference computes in fp32,
float64 where it computes in float64, wrapping uint64 for the integer fingerprints), the
algorithm of one reference function, and cites the reference file:line it follows.  Sign
patterns are drawn with torch's CPU ``Generator`` exactly as the reference draws them; the
generator itself is never reimplemented.

Modules
  lowp         bf16 / fp16 rounding of float32 values (round to nearest even)
  signs        the +-1 patterns of the signed checksum                       checksum.py:239-292
  abft         column-block check of C = beta*bias + alpha*A@B (training)   checksum.py:400-530, 695-725
  serve_check  per-layer constants and the serving check with its state row serve.py:140-244, 301-404
  fingerprint  the two integer fingerprint families (+ a C version)         recompute.py:59-116,
                                                                           serve_weights.py:73-86,151-185
  quant        int8 exact and fp8 scaled checksum checks                    modes.py:231-291
"""
