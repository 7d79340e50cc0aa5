"""CPU oracle for the paged-attention decode path — test infrastructure only.

Imported only by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg, as the checker. The product package ``simpler_amd`` never
imports it.
"""
