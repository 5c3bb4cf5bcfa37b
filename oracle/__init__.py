"""CPU oracle for the batched Householder QR path (test infrastructure only)."""
