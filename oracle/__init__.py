"""CPU oracle for the SR-SWA hot path -- test infrastructure only (see srswa_oracle)."""
