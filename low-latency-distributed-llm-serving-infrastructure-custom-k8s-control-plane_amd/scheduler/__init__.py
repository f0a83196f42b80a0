"""Request-side types the paged-attention path consumes."""
