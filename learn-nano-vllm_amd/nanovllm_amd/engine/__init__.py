"""Host-side metadata builders of the KV-cache path (mirror of nanovllm/engine)."""
