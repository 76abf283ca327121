"""CPU checker for the MoE block (test infrastructure only; see moe_oracle.h)."""
