"""CPU oracle of the KV-cache hot path — test infrastructure only (see kv_oracle.py)."""
