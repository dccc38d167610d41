"""CPU oracle for the Qwen3-0.6B decode/prefill path — TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg may
import this package, and only as the checker. The product path
(`megaqwen_amd`) never imports it.
"""
