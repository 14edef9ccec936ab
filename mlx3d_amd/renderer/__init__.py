from .protocols import Renderer, RenderOutput

__all__ = ["Renderer", "RenderOutput"]
