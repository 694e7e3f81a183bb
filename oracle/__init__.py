"""CPU oracle of the MoE hot path -- test infrastructure only (see oracle.py)."""
