"""CPU oracle of the Q38 MoE path (test infrastructure only; see moe_oracle.py)."""
