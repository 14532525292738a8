"""CPU oracle of the mHC hot path (test infrastructure only; see mhc_oracle.py)."""
