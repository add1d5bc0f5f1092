"""CPU oracle of the paged-attention hot path -- TEST INFRASTRUCTURE ONLY.

Imported only by tests/, __graft_entry__.smoke() (for the reference outputs) and
bench.py's cpu_baseline leg (as the timed CPU path).  The HIP product path in
myvllm-mini-engine_amd/ never imports it.

  paged_oracle.py  torch restatement of the reference's CPU paths
  paged_ref.c      independent C restatement (float64), built by the Makefile
  c_oracle.py      ctypes binding of the C restatement
"""
