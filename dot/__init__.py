"""Drop-in package name of the reference: ``import dot`` is ``import dot_amd``.

Everything is re-exported from :mod:`dot_amd`; ``dot._ops`` is
:mod:`dot_amd._ops` (the ``torch.ops.dot.*`` handles).
"""

import sys as _sys

import dot_amd as _impl
from dot_amd import _ops  # noqa: F401  (the reference imports _ops first)
from dot_amd import *  # noqa: F401,F403
from dot_amd import __all__, __version__  # noqa: F401

_sys.modules[__name__ + "._ops"] = _impl._ops
_sys.modules[__name__ + ".sinkhorn"] = _impl.sinkhorn
_sys.modules[__name__ + ".bidirectional_softmax"] = _impl.bidirectional_softmax
