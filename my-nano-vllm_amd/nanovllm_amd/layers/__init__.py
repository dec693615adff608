"""FP8 KV store (drop-in for store_kvcache)."""
