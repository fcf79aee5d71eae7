"""CPU oracle for the minitorch_amd hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in NumPy, what the reference (samitmohan/minitorch, pure
Python/NumPy) computes on the causal-attention / GPT-training path.  Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker.  The product
(``minitorch_amd``) never imports it and has no CPU fallback.

Modules
  attention -- the attention sub-graph, transformer.py:36-44, forward and the
               backward closures the reference's autograd runs for it.
  gpt       -- the GPT training step and greedy generation (transformer.py,
               layers.py, functional.py, loss.py, optim.py).

How each function is pinned (checked against something other than itself) is
stated in its docstring; see also tests/test_oracle.py.
"""
