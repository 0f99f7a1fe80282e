"""CPU oracle for the Mamba-2 SSD forward -- test infrastructure only.

Importable from ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg; never from the product package ``workloadsuite_amd``.
"""
