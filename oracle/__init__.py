"""TEST INFRASTRUCTURE ONLY: the CPU oracle (a C restatement of lumen/reference/mod.rs) and its graph
serializer. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it."""
