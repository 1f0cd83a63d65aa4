"""Mirror of src/matterformer/models/triton_regular_attention.py:1-3 (no fused regular attention)."""

TRITON_REGULAR_ATTENTION_AVAILABLE = False
