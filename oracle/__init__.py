"""CPU oracle (test infrastructure only): op_eager restatement, fp64 restatement, routing closed
form (eager.py) and a C restatement of routing (route.c → _build/liboracle_route.so).
Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg."""
