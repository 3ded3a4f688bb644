"""CPU oracle for the causal conv1d hot path (test infrastructure only; see oracle.py)."""
