"""CPU oracle (test infrastructure only; see asc2_oracle.py's header)."""
