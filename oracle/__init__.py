"""CPU oracle for the paged-attention hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker (or the timed CPU baseline), never as a
product path. See paged_oracle.py (numpy restatement of the reference's
algorithms) and torch_ref.py (the reference's PyTorch paths, restated, timed
as the CPU baseline).
"""
