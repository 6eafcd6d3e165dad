"""CPU oracle for the HeatKV slab-compaction + segmented-attention path.

TEST INFRASTRUCTURE ONLY.  Nothing in the ``heatkv_amd`` package imports this
package.  Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may import it, and only as the checker (or, for the
baseline, as the thing timed on the host cores) -- never as the product path.

Modules
-------
``segmented_attention``
    fp32 (or fp64) numpy restatement of ``_flat_segmented_attention_reference``
    (real_pruning_fused_attention.py:312-361), extended with the softmax
    log-sum-exp that the reference kernel does not return.
``slot_schedule``
    Line-faithful restatement of the static slab allocator
    ``_segmented_flat_build_static_slot_schedule`` and its helpers
    (enable_real_pruning_fast.py:206-558, 610-671, 1033-1047) and the policy
    lookup of ``ScaleSpecificPruningController`` (enable_pruning.py:182-189,
    380-401).
``pack``
    numpy restatement of ``_pack_flat_segments_kv_kernel``
    (real_pruning_fused_attention.py:33-73).
``produce``
    numpy restatement of the layer's QKV prologue under bf16 autocast
    (enable_real_pruning_fast.py:2040-2072: cosine-attention normalize and
    scale) and of ``apply_rotary_emb`` / ``precompute_rope2d_freqs_grid``
    (infinity/models/basic.py:39-117).

How each function is pinned (checked against something other than itself) is
stated in its own docstring; the tests under ``tests/test_oracle_*.py`` hold
the checks.
"""
