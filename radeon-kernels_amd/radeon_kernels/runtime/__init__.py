"""Static-dispatch runtime: environment fingerprint, manifests, packs, loader and explain record."""
