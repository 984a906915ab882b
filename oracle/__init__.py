"""CPU oracle of the W4A8 decode path -- test infrastructure only (see ref.py's header)."""
