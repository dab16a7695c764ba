"""CPU oracle for the neighborhood-attention hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped package imports this
directory; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker.

Contents
--------
``pure.py``
    Op-for-op restatement, in torch on the CPU, of the reference's pure
    backend (``src/natten_mps/_core/pure.py``) and of its window rule
    (``src/natten_mps/utils/window.py``).  Pinned by the golden fixtures in
    ``tests/golden/`` (written from the reference itself), by brute-force
    enumeration of windows, by the global-attention closed form and by
    float64 gradcheck (see ``tests/test_oracle_*.py``).
``window.c``
    Plain-C restatement of the window rule and of the flattened
    neighbourhood index maps (``pure.py:22-129,335-387``), built into
    ``oracle/_build/liboracle_window.so`` by ``oracle/Makefile``.  Pinned
    against ``pure.py``'s maps, the reference's known answers
    (``tests/test_shift_semantics.py:66-99``) and a brute-force
    definition of the window on tiny shapes.
"""
