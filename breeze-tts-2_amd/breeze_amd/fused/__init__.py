"""Fused RMSNorm -> GEMV -> epilogue decode path (models/fused/)."""
