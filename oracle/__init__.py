"""CPU oracle for the grad-grad attention path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or the timed
CPU baseline); the product path never calls it.

  oracle.math_path    torch restatement of the reference's math path
                      (ttt_kernels/triton_attention.py:18-25, :51-59, autograd
                      harnesses tests/bench_gradgrad.py:75-87).
  oracle.closed_form  numpy float64 closed forms: forward, first backward and
                      the full double backward.
  oracle.brute        pure-Python loops for tiny sizes, and central finite
                      differences of the looped first backward.

How each function is pinned (tests/test_oracle.py):
  * math_path.attention_math / attention_with_probs: against brute.forward
    (independent loops), special cases with textbook answers (T=1 gives V;
    q=0 gives column means of V, or prefix means when causal; causal row 0
    gives V[0]), and float64 gradcheck.
  * math_path.gradgrad_step: float64 gradgradcheck, and equality with
    closed_form.double_backward.
  * closed_form.backward: against brute.backward (loops) and torch autograd;
    the identity rowsum(P o dP) == rowsum(dO o O).
  * closed_form.double_backward: against central finite differences of
    brute.backward (independent of any autograd), and torch autograd of the
    math path; the single-pass identity for F.
  * Planted mistakes (a transposed gK term, a dropped softmax-Jacobian term,
    a wrong sign of E) are shown to fail these checks.
There are no golden vectors in the reference's tests; tests/golden holds a
C1-config fixture written by this oracle (see tests/golden/make_c1.py).
"""
