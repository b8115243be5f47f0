"""Sizing: chunk budget, arena pages, attention-path choice (quail/cost/budgets.py).

The formulas are the reference's, so a spec gives the same chunk and arena
sizes as there; MI355X is just another DeviceSpec.
"""

from quail_amd.specs import DeviceSpec, ModelSpec

POOL_FRACTION = 0.95
CHUNK_SLACK = 2
PAGE_TOKENS = 16
INT32_MAX = 2**31 - 1
ACT_BYTES = 2
ACT_RESERVE_CHUNKS = 2


def kernel_index_cap(model: ModelSpec) -> int:
    """rows x widest projection < 2^31 (budgets.py:29-34)."""
    return INT32_MAX // model.widest_projection


def chunk_memory_bound(model: ModelSpec, device: DeviceSpec) -> int:
    free = device.mem_bytes * POOL_FRACTION - model.W_resident
    return int(free // model.act_per_token) // CHUNK_SLACK


def _projection_shapes(model: ModelSpec):
    return ((model.hidden, model.qkv_width),
            (model.n_q * model.d_head, model.hidden),
            (model.hidden, model.ffn_width),
            (model.intermediate, model.hidden))


def compute_knee(model: ModelSpec, device: DeviceSpec) -> float:
    """Chunk tokens where the dense projections cross the roofline ridge."""
    ridge = device.peak_flops / device.hbm_bw
    tot_p = tot_io = 0.0
    for din, dout in _projection_shapes(model):
        tot_p += din * dout
        tot_io += din + dout
    denom = 2.0 * tot_p - ridge * tot_io * ACT_BYTES
    if denom <= 0:
        raise ValueError("projections never cross the ridge")
    return ridge * tot_p * model.w_bytes / denom


def chunk_budget(model: ModelSpec, device: DeviceSpec) -> int:
    b = min(chunk_memory_bound(model, device), kernel_index_cap(model))
    if model.chunk_cap_tokens:
        b = min(b, model.chunk_cap_tokens)
    return max(b, int(compute_knee(model, device)))


def arena_bytes(model: ModelSpec, device: DeviceSpec, chunk_tokens: int) -> float:
    return (device.mem_bytes * POOL_FRACTION - model.W_resident
            - ACT_RESERVE_CHUNKS * chunk_tokens * model.act_per_token)


def arena_pages(model: ModelSpec, device: DeviceSpec, chunk_tokens=None):
    """(every-token pages, sliding pages); no sliding layers here."""
    if chunk_tokens is None:
        chunk_tokens = chunk_budget(model, device)
    free = arena_bytes(model, device, chunk_tokens)
    return int(free // (model.kappa_full * PAGE_TOKENS)), 0


def arena_tokens(model: ModelSpec, device: DeviceSpec, chunk_tokens=None) -> int:
    full, _ = arena_pages(model, device, chunk_tokens)
    return full * PAGE_TOKENS


def _attention_time(model, device, chunk, context):
    flops = 4.0 * chunk * context * model.n_q * model.d_head
    moved = (context * model.kappa / model.layers
             + 2.0 * chunk * model.n_q * model.d_head * ACT_BYTES)
    return max(flops / device.peak_flops, moved / device.hbm_bw) * model.layers


def choose_attention_path(model: ModelSpec, device: DeviceSpec, *, readers: float,
                          reader_rows: float, node_tokens: float) -> str:
    """"unified" or "tree" for the readers of one shared node (budgets.py:179-211)."""
    if readers <= 1 or reader_rows <= 0 or node_tokens <= 0:
        return "unified"
    unified = readers * _attention_time(model, device, reader_rows, node_tokens)
    rows = readers * reader_rows
    tree = _attention_time(model, device, rows, node_tokens)
    merge = 3 * rows * model.n_q * model.d_head * ACT_BYTES / device.hbm_bw
    tree += merge * model.layers
    return "tree" if tree < unified else "unified"
