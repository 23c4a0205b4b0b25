"""CPU oracle for SparseConv2D: test infrastructure only (see sv_oracle.py)."""
