"""Native backends of the memory operator (HIP only)."""
