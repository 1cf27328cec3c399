"""CPU oracle for the SSA attention path -- test infrastructure only.

Imported only by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg, as the checker.  Never part of the product path.
"""
