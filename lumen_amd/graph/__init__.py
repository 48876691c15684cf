"""The traced graph IR, its primitives and the tracer."""
