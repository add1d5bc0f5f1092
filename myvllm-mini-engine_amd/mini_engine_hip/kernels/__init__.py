"""HIP backend entry points with the reference's kernel-dispatch signatures."""
