"""``maxsim.reference``: the pure-PyTorch functions of the reference's
torch-ext/maxsim/reference.py, as provided by :mod:`maxsim_amd.reference`."""

from maxsim_amd.reference import *  # noqa: F401,F403
from maxsim_amd.reference import __all__  # noqa: F401
