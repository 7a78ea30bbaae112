"""CPU oracle of the INT4 KV path — test infrastructure only (see kvq_oracle.py)."""
