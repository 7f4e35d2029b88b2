"""CPU oracle of the MoE-layer hot path. TEST INFRASTRUCTURE ONLY: imported by tests/, by
__graft_entry__.smoke() and by bench.py's cpu_baseline leg, never by the product package."""
