"""Oracle package — TEST INFRASTRUCTURE ONLY.

CPU restatements of HELM's paged-attention arithmetic (attention.py) and
page-management semantics (paging.py), each function citing the reference
file:line it follows.  Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import anything here, and only as the reference the
results are compared with / the timed CPU baseline.  The product package (helm_amd) never imports it.
"""
