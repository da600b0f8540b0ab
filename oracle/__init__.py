"""CPU oracle for the MENTAT branching-decode path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithm that the HIP
library replaces. Every function cites the reference file:line it follows.
It is what results are compared against, never the thing measured or
shipped: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it. The product path (``mentat_amd``) never imports it.

Modules
  attention   build_packed_kv gather + per-sequence SDPA decode (fp64 oracle
              and the reference's own torch-CPU path for the CPU baseline)
  paged_cache BlockAllocator / SequenceState / PagedKVCacheManager bookkeeping
              (set-based allocator, fork/free, lazy copy-on-write append)
  sampling    entropy, repetition penalty, gate, argmax/top-K, and the
              Philox4x32-10 temperature/top-p sampler (C, bit-exact spec)
  rollout_cpu the reference's serial rollout on the host (gather + per-sequence
              SDPA per layer), the CPU baseline of the end-to-end rollout
  build       compiles csrc/sampling_ref.c into liboracle.so

How each function is pinned (golden vectors, closed forms, library routines,
invariants) is listed in the module docstrings and exercised by
tests/test_oracle_*.py.
"""
