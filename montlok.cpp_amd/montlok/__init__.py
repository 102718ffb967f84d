"""montlok (MI355X build): the RDT4quant fused-forward path on ROCm.

``montlok._C`` holds the GPU operators under the reference's operator names;
``montlok.rdt`` holds the drop-in modules that call them.
"""

__all__ = ["rdt"]
