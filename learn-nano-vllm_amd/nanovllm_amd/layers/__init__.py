"""Layers of the KV-cache path (mirror of nanovllm/layers)."""
