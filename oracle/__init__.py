"""CPU oracle of the QSA path -- test infrastructure only (see oracle.py)."""
