"""Random-init FLUX.1-dev-architecture DiT for whole-model ConvRot measurement."""
