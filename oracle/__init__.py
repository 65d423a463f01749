"""CPU oracle of the RCSA hot path -- test infrastructure only (see rcsa_oracle)."""
