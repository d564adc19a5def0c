"""Checkpoint loading: the safetensors loader for fused AWQ layers."""
