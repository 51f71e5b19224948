"""CPU oracle of the packed refresh path — test infrastructure only (see oracle.py)."""
