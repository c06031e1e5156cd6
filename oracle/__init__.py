"""Parity oracle for the DeepSeekMoE hot path — TEST INFRASTRUCTURE ONLY.

Importable only from ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``.  Never imported by the product package.

* ``oracle.moe_ref``  torch CPU restatement of models/moe.py (float path).
* ``oracle.route``    ctypes wrapper over ``route_ref.c`` (integer routing:
                      top-k with a fixed tie rule, counts, stable permutation).
"""
