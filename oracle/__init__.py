"""CPU oracle (test infrastructure; see oracle.h)."""
