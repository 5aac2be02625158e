"""CPU oracle of the mLSTM/sLSTM kernel backend: test infrastructure only.

Imported only by ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``, as the checker (or the timed CPU
baseline).  The product package ``xlstm_hip`` never imports it.
"""
