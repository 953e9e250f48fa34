"""CPU oracle of the global-decay path — TEST INFRASTRUCTURE ONLY (see decay_oracle.py)."""
