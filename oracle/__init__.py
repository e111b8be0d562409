"""CPU oracle and CPU baseline for the SDPA forward path.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``; never by the ``tiledattention`` package.
"""
