"""CPU oracle of the kvskip decode-attention hot path -- TEST INFRASTRUCTURE ONLY.

A restatement, in float64 torch on the CPU (numpy for the integer token index), of the
reference's semantics (format37/kvskip; each function cites the file:line it follows). Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import it, and only as the
checker or the timed CPU baseline. The product (kvskip_amd/) never imports it and has no CPU
fallback.

Pinning (what makes this oracle trustworthy beyond retyping formulas) lives in
tests/test_oracle.py: library routines (torch scaled_dot_product_attention), brute-force loops on
tiny inputs, closed forms and invariants.
"""
