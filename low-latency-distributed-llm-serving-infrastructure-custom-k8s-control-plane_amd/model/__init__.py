"""Per-step / per-layer glue: step context, attention hook and backends."""
