"""CPU oracle of the projection hot path: TEST INFRASTRUCTURE ONLY (the checker for
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg). The engine in
cellerator_amd/ never imports it."""
