"""CPU oracle of the flash-attention path (test infrastructure only)."""
