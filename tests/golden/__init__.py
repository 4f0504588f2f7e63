"""Golden fixtures for the GLIF_3 cell path (inputs + expected outputs, written by the
C oracle in ``oracle/``; see ``make_golden.py``)."""
