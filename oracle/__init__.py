"""CPU oracle for the FlashAttention forward path (test infrastructure only)."""
