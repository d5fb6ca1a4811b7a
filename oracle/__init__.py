"""CPU oracle of the fused inference ops - TEST INFRASTRUCTURE ONLY.

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the checker
or the timed CPU baseline. The product (torchair_amd) never imports it.
"""
