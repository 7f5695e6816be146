"""CPU oracle of the sampling hot path (test infrastructure only; see sampling_oracle)."""
