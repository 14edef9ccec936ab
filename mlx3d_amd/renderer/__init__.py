from .protocols import Renderer, RenderOutput
from .rasterizer import Fragments, interpolate_face_attributes, rasterize_meshes

__all__ = ["Fragments", "Renderer", "RenderOutput", "interpolate_face_attributes",
           "rasterize_meshes"]
