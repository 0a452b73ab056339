"""CPU oracle package (test infrastructure only; see oracle/lx_oracle.h)."""
