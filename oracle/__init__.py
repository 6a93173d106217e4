"""CPU oracle for the palette-weight GEMM path (test infrastructure only)."""
