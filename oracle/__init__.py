"""CPU oracle for the gated delta rule.

TEST INFRASTRUCTURE ONLY.  Nothing in the product path (``avelang_amd``)
imports, links or executes anything in this directory.  Only ``tests/``,
``__graft_entry__.smoke()`` (as the checker) and the ``cpu_baseline`` leg
of ``bench.py`` may use it.

Contents
--------
``gdn_ref.py``   numpy restatement: fp64/fp32 per-token recurrence (the
                 definition) and the fp32 chunked (UT/WY) form.
``gdn_cpu.c``    C/OpenMP restatement of the same two forms, built into
                 ``oracle/_build/libgdn_oracle.so``; it is the timed CPU
                 baseline ("port") and a second, independent oracle.
``build.py``     gcc recipe for ``gdn_cpu.c``.
``layer_ref.py`` numpy restatement of the layer's neighbours of the core:
                 gating, causal conv1d (prefill and decode update), gated
                 RMSNorm, and the recurrence over a pool of state slots.

The reference tree (848267592/avelang) ships no gated-delta-rule code of
any kind (``python/avelang_kernels/`` holds only ``amdgpu_gemm.py``), so
there is no ``oracle/_ref`` build.  The restatement follows the operator
semantics of transformers' Qwen3-Next text
(``transformers/models/qwen3_next/modeling_qwen3_next.py:368-503``, read as
text) and is pinned by closed forms, invariants and textbook routines in
``tests/test_oracle.py``.
"""
