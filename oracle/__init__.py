"""CPU oracle of the MoC FFN hot path: TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import it.  The product package moc_amd/ never does.
"""
