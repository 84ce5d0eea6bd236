"""MI355X build of the reference's ``attention`` package (attention.py, triton_atopn.py)."""
