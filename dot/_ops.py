"""``dot._ops`` — the reference's low-level operator module; see :mod:`dot_amd._ops`."""

from dot_amd._ops import *  # noqa: F401,F403
from dot_amd._ops import dot, fused, _load_extension, _ensure_loaded  # noqa: F401
