"""CPU oracle of the attention path (test infrastructure only; see fqa_oracle.c)."""
