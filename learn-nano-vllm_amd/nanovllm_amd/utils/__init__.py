"""Context side channel (mirror of nanovllm/utils)."""
