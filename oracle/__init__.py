"""
oracle -- TEST INFRASTRUCTURE ONLY.

A CPU restatement of the reference WideCompiler's N-first wide forward path, written from
the reference's source (file:line cited per function).  It is the checker for the HIP
kernels of wide_compiler and nothing else: only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import it, and never as the thing measured or shipped.

* wide_ref   -- floating-point primitives, restated op-for-op in the same torch CPU ops
                and order as the reference (so bf16 rounding points match).
* bytes_ref  -- the byte / index maps (pack, boundary transpose, embedding gather) as
                closed-form numpy index arithmetic.

How each function is pinned (independently of its own formula) is listed in the module
docstrings and exercised by tests/test_oracle.py.
"""
