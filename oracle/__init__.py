"""CPU oracle for the grouped multi-LoRA apply -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker. The product path (adapterslotsplusplus_amd)
never imports it and has no CPU fallback.

  oracle.segments  -- C restatement of the segment-table rules (seg_oracle.c)
  oracle.bgmv      -- torch fp32 CPU restatement of shrink / expand / add_lora
"""
