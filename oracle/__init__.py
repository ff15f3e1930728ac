"""CPU oracle for the fused RMSNorm / SiLU-and-mul path (test infrastructure only)."""
