"""CPU oracle of the MoE feed-forward path (test infrastructure only)."""
