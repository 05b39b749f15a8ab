"""The mixers' binding to the serving engine's forward context.

Under vLLM the mixers take part in the engine's forward context as the
reference's do (mixers.py:806-829, 852-856, 1407-1410):
  * a mixer registers itself, at construction, in the current vLLM config's
    `compilation_config.static_forward_context` under its prefix (duplicate
    prefixes are refused) and adds the mixer operator to `splitting_ops`, so
    piecewise compilation splits the graph around each mixer;
  * a step's metadata is `vllm.forward_context.get_forward_context()
    .attn_metadata` (one object for every layer, or a dict keyed by prefix);
  * the operator finds its layer as `get_forward_context().no_compile_layers`
    [`_resolve_layer_name(layer_name)`], the name the layer passed through
    `_encode_layer_name(prefix)`.

Without vLLM the same three pieces are local: a registry dict, a context
object whose `attn_metadata` `set_forward_context(...)` publishes for the
duration of a step, and the lookup in the registry.  The local context also
takes precedence while it is active, so a harness can drive the mixers with
`set_forward_context` in a process where vLLM happens to be importable.
"""

import contextlib
import importlib

HYENA_MIXER_OP = "vllm::evo2_hyena_mixer"

# Layers register under their prefix here when there is no engine.
static_forward_context = {}


class ForwardContext:
    """What the mixers read from a forward context: `attn_metadata`, either
    one metadata object for every layer or a dict keyed by prefix."""

    def __init__(self):
        self.attn_metadata = None
        self.active = 0  # set_forward_context nesting depth


_context = ForwardContext()


def get_forward_context():
    """The local forward context (the engine's lives in vLLM)."""
    return _context


@contextlib.contextmanager
def set_forward_context(attn_metadata):
    """Run a model step with `attn_metadata` visible to every mixer."""
    prev = _context.attn_metadata
    _context.attn_metadata = attn_metadata
    _context.active += 1
    try:
        yield _context
    finally:
        _context.active -= 1
        _context.attn_metadata = prev


class _Engine:
    """vLLM's entry points, resolved once."""

    def __init__(self, forward_context, config, torch_utils):
        self.get_forward_context = forward_context.get_forward_context
        self.get_current_vllm_config = config.get_current_vllm_config
        self.encode = getattr(torch_utils, "_encode_layer_name", None) if torch_utils else None
        self.resolve = getattr(torch_utils, "_resolve_layer_name", None) if torch_utils else None


_UNRESOLVED = object()
_engine = _UNRESOLVED


def engine():
    """vLLM's forward-context API when vLLM imports, else None."""
    global _engine
    if _engine is _UNRESOLVED:
        try:
            fc = importlib.import_module("vllm.forward_context")
            cfg = importlib.import_module("vllm.config")
        except ImportError:
            _engine = None
        else:
            try:
                tu = importlib.import_module("vllm.utils.torch_utils")
            except ImportError:
                tu = None
            _engine = _Engine(fc, cfg, tu)
    return _engine


def reset_engine_binding():
    """Forget the resolved engine (the next call looks for vLLM again)."""
    global _engine
    _engine = _UNRESOLVED


def register_layer(prefix, layer):
    """Register a mixer under `prefix` (mixers.py:806-820)."""
    eng = engine()
    if eng is None:
        if prefix in static_forward_context:
            raise ValueError(f"Duplicate layer name: {prefix}")
        static_forward_context[prefix] = layer
        return
    comp = eng.get_current_vllm_config().compilation_config
    if prefix in comp.static_forward_context:
        raise ValueError(f"Duplicate layer name: {prefix}")
    comp.static_forward_context[prefix] = layer
    splitting = getattr(comp, "splitting_ops", None)
    if splitting is not None and HYENA_MIXER_OP not in splitting:
        splitting.append(HYENA_MIXER_OP)
    # a local step (set_forward_context) finds the layer here too
    static_forward_context[prefix] = layer


def layer_name(prefix):
    """The name the operator receives for a layer (mixers.py:826-829)."""
    eng = engine()
    if eng is not None and eng.encode is not None:
        return eng.encode(prefix)
    return prefix


def _resolve(name):
    eng = engine()
    if eng is not None and eng.resolve is not None:
        return eng.resolve(name)
    return name


def step_metadata(prefix):
    """This layer's metadata for the current step, or None (mixers.py:852-856)."""
    if _context.active or engine() is None:
        raw = _context.attn_metadata
    else:
        raw = engine().get_forward_context().attn_metadata
    if raw is None:
        return None
    return raw[prefix] if isinstance(raw, dict) else raw


def lookup_layer(name):
    """The layer the operator runs (mixers.py:1407-1410)."""
    key = _resolve(name)
    if _context.active or engine() is None:
        return static_forward_context[key]
    return engine().get_forward_context().no_compile_layers[key]
