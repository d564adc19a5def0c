"""Checkpoint loading: the safetensors loader for fused AWQ layers and a per-layer projection reader."""
