"""Parity oracle -- TEST INFRASTRUCTURE ONLY.

A CPU restatement of furiosa-opt's CPU-emulator hot path (mapping semantics in `mapping_ref`, the
`BufStorage` folds and kernel chains in `fo_cpu.c` via `emulator`). Only `tests/`,
`__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg may import it, and only as the
checker; the product library (`furiosa-opt_amd/`) never routes through it.
"""
