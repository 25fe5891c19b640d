"""CPU oracle for the silogic gate-layer hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker. The product
(:mod:`silogic_amd`) never imports it and has no CPU fallback: its compute
runs on the HIP library or raises.

Modules:

* :mod:`oracle.torch_ref` — the reference's pure-PyTorch CPU path restated as
  functions of ``(spec, state_dict, x)``: same torch ops in the same order as
  silogic/{functional,nodes,connectomes,heads,layers,models}.py, so its fp32
  values are the reference's values on the same torch build.
* :mod:`oracle.packed_ref` — numpy restatement of the reference's bit-packed
  inference semantics (silogic/bitpacking/ops.py, packed_layer.py,
  convert.py): the ``[dim, ceil(B/64)]`` int64 little-endian layout, the
  16-gate word ops, hard-parameter extraction, packed unfold / OR-pool, packed
  GroupSum.
* :mod:`oracle.lut_sim` — brute-force per-node truth-table evaluation of a
  hard FC network in pure Python/numpy loops (small cases only), restating
  silogic/fpga/circuit.py:150-248 (``extract_logic_net`` + ``simulate``).

How each function is pinned (reference golden vectors, closed forms,
brute force, invariants) is listed in the test files ``tests/test_oracle_*.py``.
Every function here has at least one such check; none is "parity unpinned".
"""
