"""Attention layer and FP8 KV store."""
