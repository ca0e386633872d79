"""Test-only CPU oracle for MaxSim (see maxsim_oracle.py).  Never imported by
the maxsim_amd package."""
