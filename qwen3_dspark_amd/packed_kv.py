"""Append-order packed KV cache: the cache state of PackedTarget and
VarlenPackedTarget (dspark_qwen/packed_target.py:30-113,
dspark_qwen/varlen_target.py:135-167) on the GPU, without the model.

Per layer, K and V are [1, H, N, D] with the rows of all requests
interleaved in append order; key_requests / key_positions (int64 [N]) name
the request marker and request-local position of every physical row.
  * append: every layer's K and V grow by the new rows in one launch
    (dspark_rows_rebuild, the reference's per-layer cat);
  * crop / remove_request: the keep mask (request != marker) | (position <
    length) becomes a stable compaction plan on the device
    (dspark_crop_plan) and every layer is rebuilt from it in one launch
    (the reference's _gather, packed_target.py:91-101), with no host sync:
    the kept row count is known on the host from the lengths;
  * layout(queries): the PackedLayout of a forward over this cache
    (VarlenPackedTarget's per-forward layout, varlen_target.py:150-167).
This is the legacy rollback path; PersistentTargetKV replaces it with
in-place commits and rollback by omission.
"""
import torch

from . import _native
from ._device import require_gfx950, upload
from .layout import PackedLayout


class AppendOrderKV:
    def __init__(self, *, layers, heads=8, dim=128, dtype=torch.bfloat16, device='cuda'):
        if any(type(n) is not int or n < 1 for n in (layers, heads, dim)):
            raise ValueError('Layers, heads and dim must be positive integers')
        if 2 * layers > 64:
            raise ValueError('At most 32 layers per cache')
        self.device = require_gfx950(device)
        _native.load()
        self.layers, self.heads, self.dim, self.dtype = layers, heads, dim, dtype
        self._elem = torch.empty((), dtype=dtype).element_size()
        if (dim * self._elem) % 16:
            raise ValueError('A KV head row must be a multiple of 16 bytes')
        self.reset()

    def reset(self):
        empty = torch.empty((1, self.heads, 0, self.dim), dtype=self.dtype, device=self.device)
        self.kv = [(empty, empty) for _ in range(self.layers)]
        self._lengths, self._markers, self._next_marker = {}, {}, 0
        self.key_requests = torch.empty(0, dtype=torch.long, device=self.device)
        self.key_positions = torch.empty_like(self.key_requests)

    @property
    def rows(self):
        return self.key_requests.numel()

    def add_request(self, request_id):
        if not isinstance(request_id, str) or not request_id or request_id in self._lengths:
            raise ValueError('Request ID must be a new nonempty string')
        self._lengths[request_id] = 0
        self._markers[request_id] = self._next_marker
        self._next_marker += 1

    @property
    def lengths(self):
        self.validate_cache()
        return dict(self._lengths)

    def marker(self, request_id):
        self._known(request_id)
        return self._markers[request_id]

    def _known(self, request_id):
        if request_id not in self._lengths:
            raise ValueError('Unknown request ID')

    def validate_cache(self, *, deep=False):
        """Host invariants (row population equals the lengths, tensor
        shapes).  deep=True also checks on the device that every request's
        positions, in physical order, are exactly 0..length-1
        (packed_target.py:76-86; one device-to-host read)."""
        total = sum(self._lengths.values())
        if self.key_requests.numel() != total or self.key_positions.numel() != total:
            raise RuntimeError('Cache marker population differs from request lengths')
        for k, v in self.kv:
            if k.shape != (1, self.heads, total, self.dim) or v.shape != k.shape:
                raise RuntimeError('Physical KV length differs from markers')
        if deep and total:
            layout_q = [m for r, m in self._markers.items() if self._lengths[r]]
            if layout_q:
                qr = torch.tensor(layout_q, dtype=torch.long, device=self.device)
                qp = torch.tensor([self._lengths[r] - 1 for r, m in self._markers.items() if self._lengths[r]],
                                  dtype=torch.long, device=self.device)
                try:
                    PackedLayout.from_metadata(qr, qp, self.key_requests, self.key_positions)
                except ValueError as e:
                    raise RuntimeError('Request positions are not exactly a cached prefix') from e

    def _rebuild(self, n_out, *, plan=None, added=None, layers=None):
        """New K/V tensors with n_out rows for `layers` (default: all): from
        `plan` (crop) or the old rows followed by `added` (append).  One
        launch for all of them."""
        layers = tuple(range(self.layers)) if layers is None else tuple(layers)
        new = [(torch.empty((1, self.heads, n_out, self.dim), dtype=self.dtype, device=self.device),
                torch.empty((1, self.heads, n_out, self.dim), dtype=self.dtype, device=self.device))
               for _ in layers]
        if n_out:
            src = [t for l in layers for t in self.kv[l]]
            dst = [t for kv in new for t in kv]
            add = None if added is None else _native.pointer_array([t for kv in added for t in kv])
            _native.call('dspark_rows_rebuild', _native.pointer_array(src), add, _native.pointer_array(dst),
                         len(dst), self.heads, self.dim * self._elem, self.rows,
                         0 if added is None else added[0][0].shape[2], None if plan is None else plan.data_ptr(),
                         n_out, _native.stream_handle(self.device))
        return new

    def _check_chunks(self, chunks):
        if not isinstance(chunks, dict) or not chunks:
            raise ValueError('Need a nonempty request-to-rows mapping')
        for r, n in chunks.items():
            self._known(r)
            if type(n) is not int or n < 1:
                raise ValueError('Each chunk needs a positive row count')
        return sum(chunks.values())

    def _check_rows(self, t, n):
        if (not isinstance(t, torch.Tensor) or t.shape != (1, self.heads, n, self.dim)
                or t.dtype != self.dtype or t.device != self.device or not t.is_contiguous()):
            raise ValueError('Appended KV must be contiguous [1, H, rows, D] of the cache dtype and device')

    def _record(self, chunks, n_new):
        """Markers and request-local positions of n_new rows appended in
        chunk order; the requests' lengths grow by their chunks."""
        markers, positions = [], []
        for r, n in chunks.items():
            markers += [self._markers[r]] * n
            positions += range(self._lengths[r], self._lengths[r] + n)
        meta = upload(self.device, markers + positions, torch.long)
        self.key_requests = torch.cat((self.key_requests, meta[:n_new]))
        self.key_positions = torch.cat((self.key_positions, meta[n_new:]))
        for r, n in chunks.items():
            self._lengths[r] += n

    @torch.no_grad()
    def append(self, chunks, projected):
        """chunks: ordered {request: new rows}; projected: per layer (keys,
        values) [1, H, sum rows, D] holding the chunks' rows in that order."""
        n_new = self._check_chunks(chunks)
        self.validate_cache()
        if len(projected) != self.layers:
            raise ValueError('Unexpected number of packed cache layers')
        for k, v in projected:
            self._check_rows(k, n_new)
            self._check_rows(v, n_new)
        self.kv = self._rebuild(self.rows + n_new, added=projected)
        self._record(chunks, n_new)

    @torch.no_grad()
    def append_layer(self, layer, keys, values):
        """Grow one layer's K and V by keys / values [1, H, n, D] (one
        launch) and return the layer's new [1, H, rows + n, D] tensors: what
        a model forward's per-layer cache update does.  commit_rows records
        the new rows once every layer has grown by them."""
        if type(layer) is not int or not 0 <= layer < self.layers:
            raise ValueError('Invalid cache layer')
        if self.kv[layer][0].shape[2] != self.rows:
            raise RuntimeError('Cache layer already grew in this forward')
        n = keys.shape[2] if isinstance(keys, torch.Tensor) and keys.ndim == 4 else -1
        self._check_rows(keys, n)
        self._check_rows(values, n)
        self.kv[layer] = self._rebuild(self.rows + n, added=[(keys, values)], layers=(layer,))[0]
        return self.kv[layer]

    def commit_rows(self, chunks):
        """Record the rows (ordered {request: rows}) by which append_layer
        grew every layer."""
        n_new = self._check_chunks(chunks)
        if any(k.shape[2] != self.rows + n_new for k, _ in self.kv):
            raise RuntimeError('Full layer cache update missing')
        self._record(chunks, n_new)

    def crop(self, request_id, length):
        """Keep one request's local prefix of `length` rows; all other rows
        stay, in order (packed_target.py:103-113)."""
        self._known(request_id)
        self.validate_cache()
        if type(length) is not int or not 0 <= length <= self._lengths[request_id]:
            raise ValueError('Crop length must be an integer within the cached request')
        if length == self._lengths[request_id]:
            return
        n = self.rows
        kept = n - (self._lengths[request_id] - length)
        plan = torch.empty(max(kept, 1), dtype=torch.long, device=self.device)
        kr = torch.empty(max(kept, 1), dtype=torch.long, device=self.device)
        kp = torch.empty(max(kept, 1), dtype=torch.long, device=self.device)
        ws = torch.empty(max(1, _native.load().dspark_crop_plan_workspace_bytes(n)), dtype=torch.uint8,
                         device=self.device)
        _native.call('dspark_crop_plan', self.key_requests.data_ptr(), self.key_positions.data_ptr(), n,
                     self._markers[request_id], length, plan.data_ptr(), kr.data_ptr(), kp.data_ptr(),
                     ws.data_ptr(), ws.numel(), _native.stream_handle(self.device))
        self.kv = self._rebuild(kept, plan=plan)
        self.key_requests, self.key_positions = kr[:kept], kp[:kept]
        self._lengths[request_id] = length

    def remove_request(self, request_id):
        """Release a finished request; a reused ID starts again at position 0."""
        self.crop(request_id, 0)
        del self._lengths[request_id], self._markers[request_id]

    def request_kv(self, request_id):
        """Per layer (keys, values) [1, H, length, D] copies in position order
        (packed_target.py:115-122); reads the request's physical rows once
        (one device-to-host sync, as the reference's nonzero)."""
        self._known(request_id)
        self.validate_cache()
        idx = torch.nonzero(self.key_requests == self._markers[request_id], as_tuple=False).flatten()
        n = idx.numel()
        out = self._rebuild(n, plan=idx) if n else self._rebuild(0)
        return tuple(out)

    def layout(self, query_requests, query_positions):
        """PackedLayout of a forward whose queries (int64 markers and
        request-local positions) are the terminal suffixes of their
        requests' cached rows (varlen_target.py:150-167)."""
        return PackedLayout.from_metadata(query_requests, query_positions, self.key_requests, self.key_positions)

    def work(self):
        """The reference's payload counter (varlen_target.py:158-166)."""
        return dict(kv_gather_payload_bytes_per_layer=self.rows * 2 * self.heads * self.dim * self._elem)
