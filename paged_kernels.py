"""Drop-in module name: nanoPD's model runner does ``import paged_kernels``
(nanoPD/engine/model_runner.py:94, :270). This re-exports the MI355X
implementation, nanopd_amd.paged_kernels."""
from nanopd_amd.paged_kernels import *  # noqa: F401,F403
from nanopd_amd.paged_kernels import __all__  # noqa: F401
