"""CPU oracle of the reference FP8 path — test infrastructure only (see fp8_oracle.py)."""
