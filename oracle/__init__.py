"""CPU oracle of the NSA selection path -- TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the checker
(or the timed CPU baseline) -- never by the omnimem_amd product path.
"""
