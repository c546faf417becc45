"""CPU oracle for the masked-attention hot path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import anything under ``oracle/``, and only as the checker (or, for the
baseline, as the timed CPU restatement).  The product package ``jaxmodules_amd``
never imports it.

Parity status of each function (what pins it) is listed in the module
docstrings and checked in ``tests/test_oracle.py``.
"""
