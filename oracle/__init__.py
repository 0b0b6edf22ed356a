"""CPU oracle of the paged-KV path (test infrastructure only)."""
