"""CPU oracle for the decode-time MoE layer (test infrastructure only; see
moe_oracle.py for who may import it)."""
