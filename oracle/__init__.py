"""CPU oracle of the cold-page codec: test infrastructure only (see oracle.py)."""
