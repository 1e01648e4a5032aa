"""CPU oracle for paged-attention decode (test infrastructure; never imported by the product)."""
