"""CPU oracle for the YABT tree-growing hot path -- test infrastructure only.

Imported by tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline
leg.  The product package (``yabt_amd``) never imports it.
"""
