"""Host optimizer of the layer-streaming path (reference optimizer/layer_adam)."""

from .layer_adam import LayerAdam  # noqa: F401
from . import cpu_adam  # noqa: F401
