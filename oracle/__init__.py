"""TEST INFRASTRUCTURE ONLY: CPU oracle (checker) for the MoE SwiGLU path.  Imported by tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg only; never by the product package."""
