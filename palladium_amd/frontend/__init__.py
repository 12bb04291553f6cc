"""A Pallas-shaped tracing frontend that needs no JAX.

`pl`, `lax`, `jnp` and `random` mirror the subset of
`jax.experimental.pallas`, `jax.lax`, `jax.numpy` and `jax.random` that
palladium kernels use, and stage the same primitives into
`palladium_amd.ir`. With JAX importable, real Pallas kernels go through
`palladium_amd.trace`'s jaxpr adapter instead.
"""

from palladium_amd.frontend import jnp, lax, pl, random
from palladium_amd.frontend.pl import ShapeDtypeStruct

__all__ = ["ShapeDtypeStruct", "jnp", "lax", "pl", "random"]
