"""CPU oracle of the batch=1 decode path -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, as the checker (or the timed CPU baseline).  The product
(cascade-llm_amd/layer_streaming) never imports it.
"""
