"""CPU oracle for the GEMM + bias + activation path (test infrastructure only)."""
