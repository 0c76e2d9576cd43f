"""CPU oracle for the GPTQ-int4 W4A16 fused-MoE path.

TEST INFRASTRUCTURE ONLY. Nothing in the product package (``mtp_amd``) may
import, call or link anything here. Only ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker or
as the timed CPU baseline, never as the thing measured on the GPU.

Modules:
  gptq_ref   unpack / dequant restated in numpy (reference
             src/mtp_expert_prefetch/repack/gptq_unpack.py:54-131)
  moe_ref    router, align/sort, expert MLP, top-k sum, shared expert, full
             layer (gptq_unpack.py:231-327, mtp/extra_tensors.py:544-598,
             tracing/vllm_router_trace.py:4178-4225)
  cache_ref  LRU slot-cache counter semantics (runtime/cache_manager.py:208-279)

Pinning (every function is checked by tests/test_oracle_*.py against the
reference's own known-answer tests, closed forms, library routines or brute
force; see each docstring).
"""
