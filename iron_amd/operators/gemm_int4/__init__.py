from .op import GEMMInt4

__all__ = ["GEMMInt4"]
