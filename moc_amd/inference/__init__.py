"""Inference-side MoC FFN: global Top-K decode and MoC 2:8 paths (moc/inference)."""
