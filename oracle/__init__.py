"""CPU oracle for the Co-ALiBi hot path (test infrastructure; see co_alibi_ref.py)."""
