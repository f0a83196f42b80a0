"""Paged KV-cache storage on the GPU: block bookkeeping, cache tensors, KV writes."""
