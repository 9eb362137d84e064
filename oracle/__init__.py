"""CPU oracle for the Qwen3 operator stack (test infrastructure: tests/, smoke(), bench CPU baseline only)."""
