"""CPU oracle for the sparse-MoE feed-forward layer.

TEST INFRASTRUCTURE ONLY. Nothing in the product path (``layerbatch_amd``) may
import this package: it is imported by ``tests/``, by ``__graft_entry__.smoke()``
as the checker, and by ``bench.py``'s CPU-baseline leg. The GPU library never
routes through it and fails loudly when its HIP build is missing.

Modules
-------
``codecs``     bf16 round-to-nearest-even and OCP e4m3fn encode/decode (numpy).
``moe``        numpy restatement of the reference MoE block
               (nanovllm/models/qwen3_5.py:754-917): router, expert permutation,
               fp32/fp64-accumulated experts, shared expert, fp8 block quantisation.
``torch_ref``  torch-CPU restatement of the reference's two expert algorithms
               (dense gather+bmm, qwen3_5.py:843-874; sparse per-expert loop,
               qwen3_5.py:815-841) with the reference's bf16 rounding points;
               timed as the CPU baseline.

Pinning status of every oracle function is listed in ``oracle/moe.py``'s header.
"""
