"""CPU oracle for the fp16 decode path: test infrastructure, never the product path."""
