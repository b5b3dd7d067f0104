"""fp64 CPU restatement of Hydra's HydraReference MoE path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package,
and only as the checker or the timed CPU baseline. The product never routes through it.
"""
