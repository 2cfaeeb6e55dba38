"""CPU restatement of the SolveDelta recurrence, used only as a test checker.

Nothing in the product path imports this package: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use it.
"""
