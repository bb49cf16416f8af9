"""CPU oracle for loom's BitNet path: test infrastructure only (see oracle.py)."""
