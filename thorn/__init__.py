"""``from thorn import THORN``: the import path of pykeio/THORN (thorn/__init__.py:1), served by the
MI355X build in ``thorn_amd``."""
from thorn_amd import THORN, THORNGroup, THORNNonOrthoGroup, THORNOrthoGroup, __version__

__all__ = ['THORN', 'THORNOrthoGroup', 'THORNNonOrthoGroup', 'THORNGroup']
