"""
Oracle for LazyLoRA's routed-expert MXFP4 path. TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package, and only as the checker or the timed CPU baseline. The product (lazylora_amd)
never imports it and never falls back to it.

Contents:
  * a float64 NumPy restatement of the path (decode, products, GLUs, router, routed
    forward/backward, the latent MoE block of the moe.json fixture);
  * ctypes access to the C restatement (mxfp4_oracle.c -> libmxfp4_oracle.so) and, when it
    was built, to the reference's own C file (oracle/_ref/libmxfp4_ref.so);
  * seeded synthetic generators for the BASELINE configurations.
"""
from .oracle import *  # noqa: F401,F403
