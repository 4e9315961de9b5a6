"""CPU oracle of the KV-cache hot path — test infrastructure only.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as
the checker. The shipped package (nanoslg_amd) never imports it.
"""
