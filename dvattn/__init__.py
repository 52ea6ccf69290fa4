"""The reference's package name, ``dvattn``, served by this build.

``import dvattn.attention`` (the reference's module, python/dvattn/attention.py)
registers ``torch.ops.libdvatt.*`` from the in-tree gfx950 library and exposes
the reference's names over this build's implementation (``dvattention_amd``).
"""
