"""CPU oracle of the encoder step (test infrastructure only)."""
