"""The engine step the paged-attention path serves: one flat forward per step."""
