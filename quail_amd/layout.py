"""Physical KV page layout of the arena, and its logical-row views.

The reference numbers arena rows page * page_tokens + slot and keeps each
layer's pool as (rows, n_kv, d) (arena.py:343-353, :519-523). quail_amd
keeps that numbering bit-exactly but stores, per layer,

  K: [n_pages, n_kv, page_tokens, d]   one 4 KiB block per (page, KV head)
  V: [n_pages, n_kv, d, page_tokens]   the same block transposed

so the attention kernel gathers a page of one KV head as one contiguous
block and reads V key-contiguous for P.V. The helpers below convert between
this layout and the reference's (rows, n_kv, d) view; they are used by
tests and diagnostics, never on the hot path.
"""

PAGE_TOKENS = 16


def k_pool_shape(n_pages, n_kv, head_dim, page_tokens=PAGE_TOKENS):
    return (n_pages, n_kv, page_tokens, head_dim)


def v_pool_shape(n_pages, n_kv, head_dim, page_tokens=PAGE_TOKENS):
    return (n_pages, n_kv, head_dim, page_tokens)


def k_paged_view(k_pool):
    """K pool as a (n_pages, page, n_kv, d) strided view (no copy)."""
    return k_pool.permute(0, 2, 1, 3)


def v_paged_view(v_pool):
    """V pool as a (n_pages, page, n_kv, d) strided view (no copy)."""
    return v_pool.permute(0, 3, 1, 2)


def k_rows(k_pool):
    """K pool as the reference's (rows, n_kv, d) view (a copy)."""
    n_pages, n_kv, page, d = k_pool.shape
    return k_pool.permute(0, 2, 1, 3).reshape(n_pages * page, n_kv, d)


def v_rows(v_pool):
    """V pool as the reference's (rows, n_kv, d) view (a copy)."""
    n_pages, n_kv, d, page = v_pool.shape
    return v_pool.permute(0, 3, 1, 2).reshape(n_pages * page, n_kv, d)


def k_pool_from_rows(rows, page_tokens=PAGE_TOKENS):
    """(rows, n_kv, d) -> K pool layout (a copy)."""
    n_rows, n_kv, d = rows.shape
    return rows.reshape(n_rows // page_tokens, page_tokens, n_kv, d) \
        .permute(0, 2, 1, 3).contiguous()


def v_pool_from_rows(rows, page_tokens=PAGE_TOKENS):
    """(rows, n_kv, d) -> V pool layout (a copy)."""
    n_rows, n_kv, d = rows.shape
    return rows.reshape(n_rows // page_tokens, page_tokens, n_kv, d) \
        .permute(0, 2, 3, 1).contiguous()


class RowPool:
    """One layer's K or V pool addressed as the reference's flat (rows, n_kv,
    d) tensor (arena.py:343-353, :851-855), over this arena's page layout.

    Row r is slot r % page_tokens of page r // page_tokens. Indexing with an
    int, a slice or a 1-D integer tensor of rows reads those rows (a copy,
    as torch's advanced indexing of the reference's pool is); assigning to
    the same indices writes through into the pages. No flat view of the
    pool exists in this layout, so slices read copies too.
    """

    def __init__(self, paged):
        self.paged = paged
        n_pages, page, n_kv, d = paged.shape
        self.page_tokens = page
        self.shape = (n_pages * page, n_kv, d)
        self.dtype = paged.dtype
        self.device = paged.device

    def __len__(self):
        return self.shape[0]

    def _rows(self, rows):
        import torch

        if isinstance(rows, int):
            rows = torch.tensor([rows])
        elif isinstance(rows, slice):
            rows = torch.arange(*rows.indices(self.shape[0]))
        elif not torch.is_tensor(rows):
            rows = torch.as_tensor(rows)
        if rows.dim() != 1 or rows.dtype.is_floating_point:
            raise IndexError("rows are an int, a slice or a 1-D integer index")
        rows = rows.to(device=self.device, dtype=torch.int64)
        if rows.numel() and (int(rows.min()) < -self.shape[0] or int(rows.max()) >= self.shape[0]):
            raise IndexError(f"row index out of range for {self.shape[0]} rows")
        rows = torch.where(rows < 0, rows + self.shape[0], rows)
        return rows // self.page_tokens, rows % self.page_tokens

    def __getitem__(self, rows):
        page, slot = self._rows(rows)
        out = self.paged[page, slot]
        return out[0] if isinstance(rows, int) else out

    def __setitem__(self, rows, value):
        page, slot = self._rows(rows)
        self.paged[page, slot] = value
