"""pth_flash_attn for MI355X: paged int8 attention (gfx950) behind the
reference's op, planner and C ABI.

Importing the package loads nothing and touches no GPU; ``pth_flash_attn.ops``
loads the op library, ``pth_flash_attn.capi`` wraps the C ABI library, and
``pth_flash_attn.planner`` is pure Python.
"""
