"""Synthetic-weight model shapes that call the region path: the Qwen3-4B-shaped
decoder (benchmark configs 3 and 4), the LFM2-1.2B-shaped hybrid (config 5) and
config 1's tiny MLP. Weights are random and seeded (no checkpoints: the
reference's loaders fetch from the HF hub, models/qwen3_4b_4bit.py:4-8), and
quantized with the build's affine rule (quantize.py)."""
