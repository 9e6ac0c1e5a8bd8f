"""CPU oracle for the W4A16 path -- test infrastructure only (see int4_oracle)."""
