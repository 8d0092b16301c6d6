"""simple_llm_amd: the KV-cache hot path of s-i-e-v-e/llm-experiments' simple-llm,
rebuilt for one MI355X (gfx950).

  gpu/          drop-in for simple-llm/src/gpu's KV-cache API over libskv.so
  model.py      the model on the cache: TransformerModel, Generator, generate_text
  backend.py    forward / sample_token / LayerParams / ModelParams with the
                signatures of simple-llm/src/jax_backend.py
  checkpoint.py the reference's model directory format (load_model, save_model)
  _lib.py       ctypes binding of the C ABI (include/skv.h)

The names a caller of the reference's backend imports
(`from jax_backend import forward, load_model, sample_token`, generate.py:5)
are importable from here; importing the package itself does not touch the GPU.
"""


def __getattr__(name):
    # lazy, so that `import simple_llm_amd` needs neither torch's GPU nor the library
    if name in ("forward", "sample_token", "LayerParams", "ModelParams", "forward_cache_clear"):
        from . import backend
        return getattr(backend, name)
    if name in ("load_model", "save_model"):
        from . import checkpoint
        return getattr(checkpoint, name)
    if name in ("generate_text", "TransformerModel", "TransformerModelParams"):
        from . import model
        return getattr(model, name)
    raise AttributeError(name)
