"""CPU oracle of the MXFP8 fused-MLP path.

TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
anything under oracle/, and only as the checker (or as the timed CPU baseline), never as the product path.

  mx_oracle.c / mx.py  -- block-32 MXFP8 quantizer, blocked scale layout, dequantization
  mlp.py               -- forward/backward of the fused SwiGLU MLP with LoRA, every bf16 rounding point kept
  lora.py              -- the LoRA epilogues beside the MLP (residual + LoRA-B)

Parity status of each function is recorded in the tests that pin it (tests/test_oracle_*.py).
"""
