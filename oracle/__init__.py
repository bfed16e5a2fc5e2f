"""CPU checker for the paged-KV decode path (test infrastructure only)."""
