"""Step metadata on the device and the bucketed decode-graph runner (the parts of nanovllm/engine that the KV-cache path needs)."""
