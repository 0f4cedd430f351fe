"""Launch layer of the gfx950 build (module path kept from the reference; no Triton inside)."""
