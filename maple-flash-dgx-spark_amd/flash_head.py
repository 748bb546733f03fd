"""FlashHead: score cluster centroids, then compute exact logits only for the
tokens of the best ``n_probes`` clusters (plus forced control tokens).

Runtime half of reference ``src/maple_run/flash_head.py``: ``FlashHead``
(:282-370) and ``build_flash_head`` (:373-463), same constructor arguments,
checkpoint tensors (``lm_head_flash.*``) and metadata (``flash_head`` in
config.json).  One call is ``ma_flash_head``: four HIP launches (centroid
GEMV, cluster selection with the -inf fill alongside, the probed rows'
GEMV scattered through ``token_map``, the forced rows) with no allocation, so
it is captured in the decode graph like the exact head.  Clustering the head
(``generate_flash_head``, the converter's k-means) is not part of the runtime.

Greedy decoding through it is exact whenever the true argmax lies in a
probed cluster or is a forced token; every logit it does produce is the
exact head's value for that token, bit for bit.  Cluster-score ties at the
cut are broken at the lower cluster index (``torch.topk`` leaves that order
unspecified).
"""

from __future__ import annotations

import torch

from . import _lib

DEFAULT_N_PROBES = 512


class FlashHead:
    """Two-phase approximate lm_head for single-stream decode."""

    def __init__(self, *, centroids_weight, centroids_scales, centroids_biases, token_map, head_weight,
                 head_scales, head_biases, force_ids, force_weight, force_scales, force_biases,
                 n_probes: int, vocab_size: int, group_size: int = 64, dtype=torch.bfloat16, device=None,
                 centroid_group_size: int | None = None):
        self.centroids_weight = centroids_weight.contiguous()
        self.centroids_scales = centroids_scales.contiguous()
        self.centroids_biases = centroids_biases.contiguous()
        self.token_map = token_map.to(torch.int32).contiguous()
        self.head_weight = head_weight.contiguous()
        self.head_scales = head_scales.contiguous()
        self.head_biases = head_biases.contiguous()
        self.n_clusters, self.cluster_size, self.nwords = (int(v) for v in self.head_weight.shape)
        if tuple(self.token_map.shape) != (self.n_clusters, self.cluster_size):
            raise ValueError(f"token_map shape {tuple(self.token_map.shape)} != "
                             f"{(self.n_clusters, self.cluster_size)}.")
        if self.centroids_weight.shape[0] != self.n_clusters:
            raise ValueError(f"{self.centroids_weight.shape[0]} centroids for {self.n_clusters} clusters.")
        self.n_probes = min(int(n_probes), self.n_clusters)
        self.group_size = int(group_size)
        self.centroid_group_size = int(centroid_group_size or group_size)
        self.vocab_size = int(vocab_size)
        tm = self.token_map
        if int(tm.min()) < 0 or int(tm.max()) >= self.vocab_size:
            raise ValueError("token_map holds ids outside the vocabulary.")
        self.force_ids = force_ids.to(torch.int32).contiguous()
        self.n_force = int(self.force_ids.numel())
        if self.n_force and (int(self.force_ids.min()) < 0 or int(self.force_ids.max()) >= self.vocab_size):
            raise ValueError("force ids outside the vocabulary.")
        self.force_weight = None if force_weight is None else force_weight.contiguous()
        self.force_scales = None if force_scales is None else force_scales.contiguous()
        self.force_biases = None if force_biases is None else force_biases.contiguous()
        dev = self.head_weight.device if device is None else torch.device(device)
        if dtype != torch.bfloat16:
            raise TypeError("the FlashHead kernels produce bf16 logits.")
        self.dtype = dtype
        self._full = torch.empty(1, 1, self.vocab_size, device=dev, dtype=dtype)
        self._cluster_ids = torch.empty(self.n_probes, device=dev, dtype=torch.int32)
        nbytes = int(_lib.load().ma_flash_head_workspace_bytes(self.n_clusters, self.n_probes))
        self._ws = torch.empty(nbytes, device=dev, dtype=torch.uint8)
        if self._ws.data_ptr() % 256:
            raise RuntimeError("workspace allocation is not 256-byte aligned")

    def __call__(self, hidden: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
        """Logits ``[1, 1, vocab]`` for the last position of ``hidden [1, T, H]``
        (or ``[1, H]``): -inf except the probed clusters' and forced tokens."""
        hv = hidden.reshape(-1, hidden.shape[-1])[-1:].contiguous()
        if hv.dtype != torch.bfloat16:
            raise TypeError("FlashHead expects bf16 hidden states.")
        if hv.shape[-1] != self.nwords * 8:
            raise ValueError(f"hidden size {hv.shape[-1]} != head K ({self.nwords * 8}).")
        full = self._full if out is None else out
        if full.numel() != self.vocab_size or full.dtype != torch.bfloat16 or not full.is_contiguous():
            raise ValueError("out must be a contiguous bf16 tensor with one entry per token.")
        cdt = _lib.dtype_code(self.centroids_scales, "centroid scales")
        hdt = _lib.dtype_code(self.head_scales, "head scales")
        fp = (lambda t: _lib.ptr(t)) if self.n_force else (lambda t: None)
        _lib.call("ma_flash_head", _lib.ptr(hv), _lib.ptr(self.centroids_weight),
                  _lib.ptr(self.centroids_scales), _lib.ptr(self.centroids_biases), cdt, self.n_clusters,
                  self.centroid_group_size, _lib.ptr(self.head_weight), _lib.ptr(self.head_scales),
                  _lib.ptr(self.head_biases), hdt, self.cluster_size, self.group_size,
                  _lib.ptr(self.token_map), self.n_probes, fp(self.force_weight), fp(self.force_scales),
                  fp(self.force_biases), fp(self.force_ids), self.n_force, self.nwords, self.vocab_size,
                  _lib.ptr(full), _lib.ptr(self._cluster_ids), _lib.ptr(self._ws), self._ws.numel(),
                  _lib.stream_of(hv))
        return full

    @property
    def cluster_ids(self) -> torch.Tensor:
        """The clusters probed by the last call (ascending)."""
        return self._cluster_ids


def build_flash_head(*, config: dict, lm_head: tuple, weights: dict, device, dtype=torch.bfloat16) -> FlashHead:
    """A ``FlashHead`` from checkpoint tensors (``weights``: the
    ``lm_head_flash.*`` entries are popped) and the exact head ``lm_head =
    (packed [V, nwords] uint32, scales, biases)``; the head's rows are
    permuted by ``token_map`` here unless the checkpoint carries the permuted
    copy (``lm_head_flash.head.*``)."""
    meta = config.get("flash_head") or (config.get("maple_run") or {}).get("flash_head")
    if not meta:
        raise ValueError("Checkpoint has no flash_head metadata; the converter attaches it.")
    if not meta.get("scaled_centroids"):
        raise ValueError("FlashHead metadata predates scaled centroids; regenerate it with the converter.")
    n_clusters = int(meta["n_clusters"])
    cluster_size = int(meta["cluster_size"])
    n_probes = int(meta.get("n_probes", DEFAULT_N_PROBES))
    group_size = int(meta.get("head_group_size", meta.get("group_size", 64)))
    centroid_group = int(meta.get("group_size", group_size))
    device = torch.device(device)
    token_map = weights.pop("lm_head_flash.token_map").to(device=device, dtype=torch.int32)
    if tuple(token_map.shape) != (n_clusters, cluster_size):
        raise ValueError(f"token_map shape {tuple(token_map.shape)} != {(n_clusters, cluster_size)} "
                         "from flash_head metadata.")
    packed, scales, biases = lm_head
    order = token_map.reshape(-1).to(torch.int64)
    if "lm_head_flash.head.weight" in weights:
        head_w = weights.pop("lm_head_flash.head.weight").to(device)
        head_s = weights.pop("lm_head_flash.head.scales").to(device)
        head_b = weights.pop("lm_head_flash.head.biases").to(device)
        if head_w.dtype != torch.uint32:
            head_w = head_w.view(torch.uint32)
        head_w = head_w.reshape(n_clusters, cluster_size, -1)
        head_s = head_s.reshape(n_clusters, cluster_size, -1).to(scales.dtype)
        head_b = head_b.reshape(n_clusters, cluster_size, -1).to(biases.dtype)
    else:
        head_w = packed.view(torch.int32).index_select(0, order).view(torch.uint32)
        head_w = head_w.reshape(n_clusters, cluster_size, -1)
        head_s = scales.index_select(0, order).reshape(n_clusters, cluster_size, -1)
        head_b = biases.index_select(0, order).reshape(n_clusters, cluster_size, -1)
    cw = weights.pop("lm_head_flash.centroids.weight").to(device)
    if cw.dtype != torch.uint32:
        cw = cw.view(torch.uint32)
    # centroid scales and biases in bf16, as the head's (reference model.py:728-748)
    cs = weights.pop("lm_head_flash.centroids.scales").to(device=device, dtype=scales.dtype)
    cb = weights.pop("lm_head_flash.centroids.biases").to(device=device, dtype=biases.dtype)
    weights.pop("lm_head_flash.cluster_scale", None)
    vocab = int(config["vocab_size"])
    force = [int(t) for t in meta.get("force_tokens", []) if 0 <= int(t) < vocab]
    if force:
        fid = torch.tensor(force, device=device, dtype=torch.int64)
        fw = packed.view(torch.int32).index_select(0, fid).view(torch.uint32)
        fs, fb = scales.index_select(0, fid), biases.index_select(0, fid)
    else:
        fid = torch.empty(0, device=device, dtype=torch.int64)
        fw = fs = fb = None
    return FlashHead(centroids_weight=cw, centroids_scales=cs, centroids_biases=cb, token_map=token_map,
                     head_weight=head_w, head_scales=head_s, head_biases=head_b, force_ids=fid,
                     force_weight=fw, force_scales=fs, force_biases=fb, n_probes=n_probes, vocab_size=vocab,
                     group_size=group_size, dtype=dtype, device=device, centroid_group_size=centroid_group)
