"""CPU oracle of the attention contract (test infrastructure only)."""
