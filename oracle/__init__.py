"""CPU oracle for the W4A16 qlinear and routed-MoE expert FFN.

TEST INFRASTRUCTURE ONLY.  This package is the oracle the tests check against: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The product path (``qwen3.5-35b-dflash_amd``) never imports, links
or falls back to anything here.

It restates, on the CPU, the arithmetic of the reference's hot path:

* ``oracle.w4``       -- portable K-packed int4 format, group quantizer,
                         dequantisation and the W4A16 linear
                         (``model/qwen35_moe_dflash/graph/quant_weights.py:124-148``,
                         ``graph/quant_plan.py:76-87``,
                         ``target/layer_probe/qlinear_math.py:73-118``).
* ``oracle.routing``  -- router softmax top-k with renormalised weights and the
                         stable token-to-expert permutation
                         (``reference/fused_ops.py:160-164``,
                         ``graph/fused/quant_target.py:168-172``,
                         ``fused/quantization.py:184-191``).
* ``oracle.moe``      -- expert FFN (gate/up, SiLU*up, down), weighted combine
                         and the gated shared expert
                         (``reference/fused_ops.py:165-173``,
                         ``target/prefill_t64/cpu_reference.py:160-181``,
                         ``fused/model.py:296-307``).
* ``oracle.metrics``  -- fp64 comparison metrics
                         (``common/accuracy.py:49-127``).

Pinning status of every function is stated in its module docstring; the tests
under ``tests/test_oracle_*.py`` hold the checks (golden vectors written by an
independent pure-Python brute force, closed forms, library routines and
invariants).
"""
