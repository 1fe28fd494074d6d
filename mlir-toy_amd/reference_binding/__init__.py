"""Reference-side bindings: modules a maintainer of the reference adds to it
(under src/neptune_mlir/backends/) to launch this backend. They are kept
here so the CPU suite can import and check them."""
