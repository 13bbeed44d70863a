"""CPU oracle for the Qwen3-VL vision tower (`encode_vision`): TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import
this package, and only as the checker (or the timed CPU baseline). The product path under
`qwen3-vl-jax_amd/` never imports it and fails loudly when its HIP library is missing.

Modules
-------
indices       integer metadata (cu_seqlens, rotary (h,w) ids, pos-embed taps, merge rows),
              restated from the reference's own reshape/repeat chains, plus the closed forms
              used as an independent cross-check.
vision_tower  the tower forward (patch embed, pos-embed, rotary, blocks, mergers) in numpy,
              in three precisions: "fp64" (exact maths), "fp32" (the reference's default dtype)
              and "bf16" (the reference's bf16 mode, rounding at the same points).
torch_tower   the same forward with torch-CPU kernels (fp32 / bf16): the CPU baseline that
              bench.py times; pinned against vision_tower.

Pin status (what checks each function, beyond retyping it):
  indices.*                   closed forms (Appendix-A style) on every grid up to 8x8x3 frames;
                              transformers' `vision_utils` helpers (t=1 and, for the ids and
                              cu_seqlens, t>1).
  layer_norm / gelu_tanh      torch.nn.functional.layer_norm / gelu(approximate="tanh") in fp64.
  attention_varlen            torch scaled_dot_product_attention per segment in fp64; softmax row
                              sums, key-permutation invariance, no cross-segment leakage, L=1 -> v.
  apply_rotary                complex-multiplication restatement of the neox pairing.
  encode_vision (fp64)        transformers' Qwen3VLVisionModel in float64 with the same weights
                              (merger activation set to tanh-GELU, as jax.nn.gelu's default is),
                              fed the reference's pos-embed taps for t>1 grids.
  bf16 rounding points        apply_rotary, pos_embed, dense and the residual adds: against torch-CPU
                              bf16 ops written op by op as the reference writes them in eager jnp
                              (each op rounds; bit-exact, dense within one product ulp), each with a
                              planted single-rounding mistake that the check catches
                              (tests/test_oracle_bf16.py). Still "parity unpinned" at the ulp
                              level: gelu (jax.nn.gelu is jitted; whether XLA:CPU rounds its bf16
                              intermediates cannot be checked without jax) and XLA's f32 exp/tanh.
  torch_tower                 vision_tower in fp32 (rel-L2 1e-5) and bf16 (1e-2), plus a planted
                              rotate_half mistake (tests/test_oracle_torch.py).
"""
