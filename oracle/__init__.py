"""CPU oracle for the quantized DiT linear path — TEST INFRASTRUCTURE ONLY.

A restatement, on the CPU, of the reference's arithmetic for each function on
the path (each function cites the reference file:line it follows).  Only
tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may import or
run anything here, and only as the checker or the timed CPU baseline — never
as the product path.  The product (xgen_amd) has no CPU implementation.

Parity pinning (what each oracle function is checked against) is listed in
the docstring of oracle/ref.py; the checks live in tests/test_oracle_*.py.
"""
