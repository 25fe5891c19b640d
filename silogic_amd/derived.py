"""Per-module caches of tables derived from the parameters.

A forward without gradients reduces the parameters to device tables before
its kernels run: soft records (resolved taps, softmax weights, node
coefficients), hard codes (argmax gates as truth tables). For a model whose
weights do not change between calls these tables are the same every time,
so they are kept on the module and rebuilt only when one of the tensors they
come from changes. The key of a table is the storage address and version
counter of every parameter and buffer of the modules it reads: in-place
updates (optimizer steps, ``copy_``, ``load_state_dict``) bump the version,
and moving or replacing a tensor changes its storage. Writes through
``tensor.data`` bypass the version counter; call :func:`clear` on a model
after such writes. Tracing under ``torch.compile`` builds the tables afresh.
"""
import torch

# Module structure generation: bumped whenever any module registers a child
# module (attribute assignment, add_module, ModuleList appends: the global
# registration hook below), which is how a model's set of parameter and
# buffer dictionaries can change. Parameters and buffers themselves may be
# replaced freely (Module._apply writes new buffers straight into
# ``_buffers``): the key reads the dictionaries' current values every time.
_structure = [0]


def _module_registered(module, name, submodule):
    _structure[0] += 1
    return None


torch.nn.modules.module.register_module_module_registration_hook(_module_registered)


def _tensors(m, out):
    out.extend(m._parameters.values())
    out.extend(m._buffers.values())
    for child in m._modules.values():
        if child is not None:
            _tensors(child, out)


def _dicts(m, out):
    out.append(m._parameters)
    out.append(m._buffers)
    for child in m._modules.values():
        if child is not None:
            _dicts(child, out)


def _module_dicts(m):
    """The parameter and buffer dictionaries of ``m`` and its submodules,
    kept on ``m`` until any module registers a child module."""
    ent = m.__dict__.get("_derived_dicts")
    if ent is None or ent[0] != _structure[0]:
        ds = []
        _dicts(m, ds)
        ent = (_structure[0], ds)
        m.__dict__["_derived_dicts"] = ent
    return ent[1]


def state_key(*modules):
    """Storage and version of every parameter and buffer of ``modules`` (this
    runs on every forward: the module tree's dictionaries are walked from a
    list kept per module, their tensors read afresh)."""
    # device allocations have distinct addresses across devices (one
    # virtual address space), so the pointer also tells the device apart
    return tuple((t.data_ptr(), t._version)
                 for m in modules for d in _module_dicts(m) for t in d.values()
                 if t is not None)


def cached(owner, name, key, build):
    """``build()``'s result, kept on ``owner`` under ``name`` while ``key``
    (from :func:`state_key` plus the call's shapes) stays the same."""
    if torch.compiler.is_compiling():
        return build()
    slot = owner.__dict__.get(name)
    if slot is not None and slot[0] == key:
        return slot[1]
    value = build()
    owner.__dict__[name] = (key, value)
    return value


def clear(model):
    """Drop every cached table of ``model`` and its submodules."""
    for m in model.modules():
        for name in [n for n in m.__dict__ if n.startswith("_derived_")]:
            del m.__dict__[name]
