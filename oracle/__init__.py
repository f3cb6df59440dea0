"""CPU oracle and CPU baseline — test infrastructure only (see cce_oracle.py)."""
