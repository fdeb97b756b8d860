"""CPU parity oracle for causal RACE attention -- TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, as the checker. The product package (race_attention_amd) never imports,
links or executes anything here.
"""
