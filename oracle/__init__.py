"""CPU oracle for the tensor-op library: test infrastructure only (see oracle.py)."""
