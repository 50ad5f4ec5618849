"""CPU oracle for the training_dynamic transformer step — TEST INFRASTRUCTURE ONLY.

This package is a plain fp32 numpy restatement of the reference's training step
(forward, backward, cross-entropy, AdamW, clip, LR schedule), of its KV-cached
token loop (tools/generate.py) and of its v4 checkpoint format.  Only the test
suite, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py``
may import it, and only as the checker.  The product path (libne.so, the ``train``
CLI, the ctypes wrapper) never calls into it.

Parity pins (what each function is checked against, see tests/test_oracle_*.py):

* forward / loss     - token-by-token KV-cached loop restated from generate.py
                       (independent code path), golden vectors written by
                       tests/golden/make_generate_vectors.py, closed form
                       loss = ln V at zero weights.
* backward           - float64 torch autograd of an independent torch model,
                       central finite differences on a tiny model.
* rmsnorm            - closed form x = c*1  ->  y = g*c/sqrt(c^2+eps).
* rope               - identity at position 0, norm preservation, closed-form
                       rotation angle pos*theta^(-2i/hd).
* AdamW              - closed form at t=1: w1 = w0 - lr*(g/(|g|+eps) + wd*w0).
* clip / LR schedule - closed forms.
* checkpoint v4      - hand-built header with known field offsets, byte-exact
                       round trip.
"""
