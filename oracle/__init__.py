"""CPU oracle for the FP8 paged-attention hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this
package; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may use it, and only as the checker
(or, in the bench, as the timed CPU baseline).

Modules:
  fp8        -- closed-form RNE E4M3FN quantisation (numpy), the 65,536-entry
                bf16 -> e4m3 table, exact dequantisation.
  attention  -- torch-CPU restatement of the reference's paged decode and
                varlen causal prefill (paged and contiguous), including the
                fp32 -> fp16 -> bf16 output rounding.
  metadata   -- pure-Python restatement of the model runner's slot-mapping,
                cu_seqlens and block-table construction.
"""
