"""CPU oracle for the mHC-lite path: test infrastructure only (see mhc_oracle)."""
