"""Drop-in import name: ``import mtlattn`` resolves to the MI355X build.

Everything (including the ``_C`` binding used by the reference's tests,
tests/test_correctness.py:356) is re-exported from ``mtlattn_amd``.
"""

from mtlattn_amd import *  # noqa: F401,F403
from mtlattn_amd import __all__, __version__, _C  # noqa: F401
from mtlattn_amd import _basic_ok, _prep_bias, _sdpa_mask_to_bias, _try_padding_varlen  # noqa: F401
# beyond the reference's API (kept out of __all__, which matches it)
from mtlattn_amd import paged_decode  # noqa: F401
