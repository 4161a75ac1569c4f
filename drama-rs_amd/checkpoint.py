"""Loader for the MoE weights of a converted drama-rs checkpoint ("drama-rs-v1").

Reads the directory layout the reference's converter writes and its Rust loader reads
(tools/convert.py:224-263,345-346; src/model.rs:186-291): ``drama.json`` (format name, int4
and int8 group sizes, the model config) and one ``layerNN.safetensors`` per decoder layer with

    post_norm                 f32  [H]             RMSNorm weight of the MoE input (+1 folded in)
    moe.router                bf16 [E + 1, H]      router rows, row E = shared-expert gate
    moe.gate_up.q4 / .sm      u8 [E, 2I, H/2] / f16 [E, 2I, H/64, 2]
    moe.down.q4 / .sm         u8 [E, H, I/2]  / f16 [E, H, I/64, 2]
    moe.shared_gate_up.q8/.s  i8 [2I, H]      / f16 [2I, H/128]
    moe.shared_down.q8 / .s   i8 [H, I]       / f16 [H, I/128]

Only the MoE tensors are read (attention, DeltaNet and the audio tower are outside this
library).  Dtypes and shapes are checked the way src/model.rs:193-230 checks them, with the
same "layerNN.name: dtype X, expected Y" style errors.  ``MoeStack`` uploads the layers to the
GPU and drives the fused decode step (dr_moe_decode_step, reference f16 formats), the
per-layer chain (dr_router_topk + dr_moe_decode) or the chunked prefill over them.
"""
from __future__ import annotations

import json
import os

import dramamoe

FORMAT = "drama-rs-v1"
Q4_GROUP, Q8_GROUP = 64, 128
LL_WORDS = dramamoe.STEP_LL_WORDS


class CheckpointError(ValueError):
    pass


def read_meta(path: str) -> dict:
    with open(os.path.join(path, "drama.json")) as f:
        meta = json.load(f)
    if meta.get("format") != FORMAT or meta.get("q4_group") != Q4_GROUP or meta.get("q8_group") != Q8_GROUP:
        raise CheckpointError(f"unsupported converted format in {path}")
    tc = meta["config"]["text_config"]
    for k in ("hidden_size", "num_hidden_layers", "num_experts", "num_experts_per_tok", "moe_intermediate_size"):
        if k not in tc:
            raise CheckpointError(f"drama.json: text_config.{k} missing")
    return meta


def _expect(prefix, name, t, dtype, shape):
    import torch

    if t.dtype != dtype:
        raise CheckpointError(f"{prefix}{name}: dtype {t.dtype}, expected {dtype}")
    if tuple(t.shape) != tuple(shape):
        raise CheckpointError(f"{prefix}{name}: shape {tuple(t.shape)}, expected {tuple(shape)}")
    return t.contiguous() if isinstance(t, torch.Tensor) else t


def read_layer(path: str, i: int, tc: dict, experts: bool = True) -> dict:
    """Host tensors (torch, CPU) of layer i's MoE, checked against the config; experts=False
    skips the int4 routed experts (when they come from an FP8 source)."""
    import torch
    from safetensors import safe_open

    H, E, I = tc["hidden_size"], tc["num_experts"], tc["moe_intermediate_size"]
    prefix = f"layer{i:02d}."
    fn = os.path.join(path, f"layer{i:02d}.safetensors")
    out = {}
    with safe_open(fn, framework="pt", device="cpu") as f:
        names = set(f.keys())

        def get(name, dtype, shape):
            if name not in names:
                raise CheckpointError(f"{prefix}{name}: not in {os.path.basename(fn)}")
            return _expect(prefix, name, f.get_tensor(name), dtype, shape)

        out["nw"] = get("post_norm", torch.float32, (H,))
        out["router"] = get("moe.router", torch.bfloat16, (E + 1, H))
        if experts:
            out["gu_q"] = get("moe.gate_up.q4", torch.uint8, (E, 2 * I, H // 2))
            out["gu_s"] = get("moe.gate_up.sm", torch.float16, (E, 2 * I, H // Q4_GROUP, 2))
            out["d_q"] = get("moe.down.q4", torch.uint8, (E, H, I // 2))
            out["d_s"] = get("moe.down.sm", torch.float16, (E, H, I // Q4_GROUP, 2))
        out["sgu_q"] = get("moe.shared_gate_up.q8", torch.int8, (2 * I, H))
        out["sgu_s"] = get("moe.shared_gate_up.s", torch.float16, (2 * I, H // Q8_GROUP))
        out["sd_q"] = get("moe.shared_down.q8", torch.int8, (H, I))
        out["sd_s"] = get("moe.shared_down.s", torch.float16, (H, I // Q8_GROUP))
    return out


def write_layer(path: str, i: int, tensors: dict) -> None:
    """Write layer i's MoE tensors under the reference's names (for tests and tools that make
    synthetic checkpoints); ``tensors`` uses the keys read_layer returns."""
    from safetensors.torch import save_file

    names = {"nw": "post_norm", "router": "moe.router", "gu_q": "moe.gate_up.q4", "gu_s": "moe.gate_up.sm",
             "d_q": "moe.down.q4", "d_s": "moe.down.sm", "sgu_q": "moe.shared_gate_up.q8",
             "sgu_s": "moe.shared_gate_up.s", "sd_q": "moe.shared_down.q8", "sd_s": "moe.shared_down.s"}
    save_file({names[k]: v.contiguous() for k, v in tensors.items()}, os.path.join(path, f"layer{i:02d}.safetensors"))


def write_meta(path: str, H: int, E: int, I: int, layers: int, topk: int = 8, eps: float = 1e-6) -> None:
    tc = {"hidden_size": H, "num_hidden_layers": layers, "num_experts": E, "num_experts_per_tok": topk,
          "moe_intermediate_size": I, "shared_expert_intermediate_size": I, "rms_norm_eps": eps}
    with open(os.path.join(path, "drama.json"), "w") as f:
        json.dump({"format": FORMAT, "q4_group": Q4_GROUP, "q8_group": Q8_GROUP, "config": {"text_config": tc}}, f,
                  indent=1)


FP8_BLOCK = 128


class Fp8Source:
    """Routed experts in their original block-FP8 form, read from the source checkpoint (the
    reference's Fp8Source, src/model.rs:406-506): ``model.safetensors.index.json`` maps every
    tensor to its shard; expert ex of layer li is

        model.language_model.layers.{li}.mlp.experts.{ex}.{gate,up,down}_proj.weight
            F8_E4M3 [I, H] (gate, up) / [H, I] (down)
        ....weight_scale_inv   F32 [rows / 128, cols / 128]

    ``layer`` assembles the layouts the FP8 kernels take (src/model.rs:99-100): gate_up w
    [E, 2I, H] (gate rows, then up rows) with s [E, 2I/128, H/128], down w [E, H, I] with
    s [E, H/128, I/128]; dtypes and shapes are checked with the reference's messages."""

    def __init__(self, path: str):
        fn = os.path.join(path, "model.safetensors.index.json")
        try:
            with open(fn) as f:
                self.weight_map = json.load(f)["weight_map"]
        except (OSError, KeyError, ValueError) as e:
            raise CheckpointError(f"read {fn}: {e}") from None
        self.path = path

    def layer(self, li: int, E: int, H: int, I: int) -> dict:
        import torch
        from safetensors import safe_open

        B = FP8_BLOCK
        if H % B or I % B:
            raise CheckpointError(f"fp8 experts: hidden {H} / intermediate {I} not a multiple of {B}")
        prefix = f"model.language_model.layers.{li}.mlp.experts"
        out = {"gu_q": torch.empty(E, 2 * I, H, dtype=torch.uint8), "gu_s": torch.empty(E, 2 * I // B, H // B),
               "d_q": torch.empty(E, H, I, dtype=torch.uint8), "d_s": torch.empty(E, H // B, I // B)}
        handles = {}
        try:
            def get(ex, part, scale, rows, cols):
                name = f"{prefix}.{ex}.{part}.weight" + ("_scale_inv" if scale else "")
                shard = self.weight_map.get(name)
                if shard is None:
                    raise CheckpointError(f"{name} not in the checkpoint index")
                if shard not in handles:
                    handles[shard] = safe_open(os.path.join(self.path, shard), framework="pt", device="cpu")
                f = handles[shard]
                if name not in f.keys():
                    raise CheckpointError(f"{name}: not in {shard}")
                t = f.get_tensor(name)
                dt, shape = (torch.float32, (rows // B, cols // B)) if scale else (torch.float8_e4m3fn, (rows, cols))
                if t.dtype != dt or tuple(t.shape) != shape:
                    raise CheckpointError(f"{name}: {t.dtype} {tuple(t.shape)}, expected {dt} {shape}")
                return t.view(torch.uint8) if not scale else t

            for ex in range(E):
                out["gu_q"][ex, :I] = get(ex, "gate_proj", False, I, H)
                out["gu_q"][ex, I:] = get(ex, "up_proj", False, I, H)
                out["gu_s"][ex, :I // B] = get(ex, "gate_proj", True, I, H)
                out["gu_s"][ex, I // B:] = get(ex, "up_proj", True, I, H)
                out["d_q"][ex] = get(ex, "down_proj", False, H, I)
                out["d_s"][ex] = get(ex, "down_proj", True, H, I)
        finally:
            handles.clear()
        return out


_KEYS = ("router", "nw", "gu_q", "gu_s", "d_q", "d_s", "sgu_q", "sgu_s", "sd_q", "sd_s")  # dr_decode_layer order
_EXPERT_KEYS = ("gu_q", "gu_s", "d_q", "d_s")


class MoeStack:
    """The MoE layers of a converted checkpoint on the GPU.

    With ``fp8_dir`` the routed experts come from the original block-FP8 checkpoint instead
    of the int4 tensors (the reference's ExpertMode::Fp8, src/model.rs:252-288): layers below
    ``vram_layers`` (all when None) are uploaded to the GPU, the others stay in pinned host
    memory that the kernels read over PCIe (src/model.rs:81-97).

    ``pack_prefill`` keeps a second copy of each layer's routed experts in the tile-step layout
    of dr_moe_pack_q4 (dr_moe_pack_fp8 for fp8 experts, whose scales are shared), which prefill
    reads (the same results, less time; the int4 copy is as large as the experts, 6% of an
    MI355X's HBM for 40 layers).  fp8 layers left in host memory are not packed."""

    def __init__(self, path: str, layers: list[int] | None = None, device: str = "cuda", fp8_dir: str | None = None,
                 vram_layers: int | None = None, pack_prefill: bool = False):
        import torch

        meta = read_meta(path)
        self.tc = tc = meta["config"]["text_config"]
        self.H, self.E, self.I = tc["hidden_size"], tc["num_experts"], tc["moe_intermediate_size"]
        self.topk = tc["num_experts_per_tok"]
        self.eps = float(tc.get("rms_norm_eps", 1e-6))
        self.fp8 = fp8_dir is not None
        ids = list(range(tc["num_hidden_layers"])) if layers is None else list(layers)
        src = Fp8Source(fp8_dir) if self.fp8 else None
        self.layers = []
        for i in ids:
            h = read_layer(path, i, tc, experts=not self.fp8)
            L = {k: v.to(device) for k, v in h.items()}
            if src is not None:
                ex = src.layer(i, self.E, self.H, self.I)
                on_gpu = vram_layers is None or i < vram_layers
                L.update({k: (v.to(device) if on_gpu else v.pin_memory()) for k, v in ex.items()})
            self.layers.append(L)
        tab = [[L[k].data_ptr() for k in _KEYS] for L in self.layers]
        self.table = torch.tensor(tab, dtype=torch.int64, device=device)
        self.ll = torch.zeros(LL_WORDS, dtype=torch.int64, device=device)
        self.sync = torch.zeros(4, dtype=torch.int32, device=device)
        self.lib = dramamoe.lib()
        self.packed = []  # per layer: the routed experts in the tile-step layout (pack_prefill)
        if pack_prefill:
            P = dramamoe.ptr
            for L in self.layers:
                if self.fp8 and not L["gu_q"].is_cuda:
                    self.packed.append(None)
                    continue
                pk = dict(L) if self.fp8 else {}
                for q, sc, n, k in (("gu_q", "gu_s", 2 * self.I, self.H), ("d_q", "d_s", self.H, self.I)):
                    pk[q] = torch.empty_like(L[q])
                    if self.fp8:
                        rc = self.lib.dr_moe_pack_fp8(P(L[q]), self.E, n, k, P(pk[q]), dramamoe.stream_ptr())
                    else:
                        pk[sc] = torch.empty_like(L[sc])
                        rc = self.lib.dr_moe_pack_q4(P(L[q]), P(L[sc]), self.E, n, k, P(pk[q]), P(pk[sc]),
                                                     dramamoe.stream_ptr())
                    if rc != 0:
                        raise ValueError(f"expert shape {n}x{k} has no tile-step layout")
                self.packed.append(pk)
            torch.cuda.synchronize()
        self._gemm = {}  # stream handle -> GEMM handle (one per stream for the stack's lifetime)

    def _gemm_handle(self, st) -> int:
        import ctypes

        key = int(st or 0)
        if key not in self._gemm:
            h = ctypes.c_void_p()
            self.lib.dr_cublas_create(ctypes.byref(h), st)  # raises DramaMoeError on a nonzero return
            if not h.value:
                raise dramamoe.DramaMoeError("dr_cublas_create returned a null handle")
            self._gemm[key] = h.value
        return self._gemm[key]

    def close(self) -> None:
        """Releases the GEMM handles created per stream (the tensors go with the object)."""
        for h in self._gemm.values():
            self.lib.dr_cublas_destroy(h)
        self._gemm.clear()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def step(self, x, stream=None, idx_out=None, wts_out=None, sgate_out=None, xs_out=None) -> None:
        """x (f32 [H], device) through every loaded layer in one fused launch, in place."""
        P = dramamoe.ptr
        f = self.lib.dr_moe_decode_step_fp8 if self.fp8 else self.lib.dr_moe_decode_step
        f(P(self.table), len(self.layers), P(x), self.E, self.H, self.I, self.topk, self.eps, P(self.ll), P(self.sync),
          P(idx_out), P(wts_out), P(sgate_out), P(xs_out), None, 0, stream if stream is not None else dramamoe.stream_ptr())
        if int(self.sync[1].item()) != 0:
            raise dramamoe.DramaMoeError("dr_moe_decode_step timed out waiting for its workgroups")

    def prefill(self, l: int, x, hn, chunk: int = 1024, stream=None, keep: dict | None = None) -> None:
        """Prefill of loaded layer l for rows token rows (the engine's moe_prefill,
        src/engine.rs:544-604): x f32 [rows, H] residual stream updated in place, hn bf16
        [rows, H] its RMSNorm.  Rows go in chunks of at most `chunk` (grouping handles up to
        8192 (row, expert) pairs per call): router GEMM, top-k, device-side grouping, gather,
        grouped expert GEMMs and the weighted combine, with the shared expert on a second stream
        beside them; no host round trip.  With ``keep`` (a dict), the last chunk's routing
        (idx, wts, sgate), grouping (slot_of) and bf16 activations (act in grouped-slot order,
        sact per row) are left in it for inspection."""
        import torch

        P = dramamoe.ptr
        L, lib = self.layers[l], self.lib
        st = stream if stream is not None else dramamoe.stream_ptr()
        rows = x.shape[0]
        H, E, I, k = self.H, self.E, self.I, self.topk
        if chunk * k > 8192:
            raise ValueError("chunk * topk must be <= 8192 (the pairs dr_moe_topk_group sorts in one call)")
        c = min(chunk, rows)
        dev = x.device
        # temporaries come from the caching allocator of the stream the kernels run on, so they
        # are not handed out again while this call's kernels are pending on it; the side stream
        # waits for `main` before it touches them and `main` waits for it before the combine
        main = torch.cuda.ExternalStream(st) if int(st) != 0 else torch.cuda.current_stream(dev)
        with torch.cuda.stream(main):
            z = lambda n, dt=torch.float32: torch.empty(n, dtype=dt, device=dev)
            logits, idx, wts, sg = z(c * (E + 1)), z(c * k, torch.int32), z(c * k), z(c)
            sact, sh = z(c * I, torch.int16), z(c * H)
            counts, offsets, slot_of = z(E, torch.int32), z(E, torch.int32), z(c * k, torch.int32)
            row_of_slot, counter = z(c * k + 16, torch.int32), torch.zeros(4, dtype=torch.int32, device=dev)
            act, yp = z(c * k * I, torch.int16), z(c * k * H)
        gh = self._gemm_handle(st)
        # the shared expert needs only hn, so it runs on a second stream beside the routing and
        # grouping and joins before the combine.  Only from a created stream: events
        # recorded through a wrapper of the null stream (handle 0) did not order the kernels
        # launched on it (measured: chunk k + 1's shared output overwrote chunk k's before its
        # combine), so on the null stream everything stays in order on it.
        overlap = int(st) != 0 and c >= 64  # for a few rows the events cost more than they save
        if overlap:
            side = torch.cuda.Stream(device=dev)
            fork, join = torch.cuda.Event(), torch.cuda.Event()
        for r0 in range(0, rows, c):
            n = min(c, rows - r0)
            hr, xr = hn[r0:r0 + n], x[r0:r0 + n]
            if overlap:
                fork.record(main)
                side.wait_event(fork)
            lib.dr_moe_shared_prefill(P(L["sgu_q"]), P(L["sgu_s"]), P(L["sd_q"]), P(L["sd_s"]), P(hr), n, P(sact),
                                      P(sh), H, I, side.cuda_stream if overlap else st)
            if overlap:
                join.record(side)
            lib.dr_gemm(gh, P(hr), P(L["router"]), P(logits), n, E + 1, H, 0.0)
            # top-k and the grouping in one launch; the grouped GEMM reads its token rows from hn
            # through row_of_slot (no gathered copy)
            lib.dr_moe_topk_group(P(logits), n, E, k, E + 1, P(idx), P(wts), P(sg), P(counts), P(offsets),
                                  P(slot_of), P(row_of_slot), P(counter), st)
            W = self.packed[l] if self.packed and self.packed[l] is not None else L
            if self.fp8:
                pf = lib.dr_moe_prefill_rows_packed_fp8 if W is not L else lib.dr_moe_prefill_rows_fp8
            else:
                pf = lib.dr_moe_prefill_rows_packed if W is not L else lib.dr_moe_prefill_rows
            pf(P(W["gu_q"]), P(W["gu_s"]), P(W["d_q"]), P(W["d_s"]), P(hr), n, P(row_of_slot), P(offsets), P(counts),
               P(act), P(yp), E, H, I, st)
            if overlap:
                main.wait_event(join)
            lib.dr_moe_combine(P(xr), P(yp), P(slot_of), P(wts), P(sg), P(sh), n, k, H, st)
        if keep is not None:
            keep.update({"idx": idx[:n * k], "wts": wts[:n * k], "sgate": sg[:n], "slot_of": slot_of[:n * k],
                         "act": act[:n * k * I], "sact": sact[:n * I]})

    def chain(self, x, stream=None) -> None:
        """The same layers through the engine's per-layer launches (router, then decode)."""
        import torch

        P = dramamoe.ptr
        st = stream if stream is not None else dramamoe.stream_ptr()
        dev = x.device
        logits = torch.empty(self.E + 1, device=dev)
        idx = torch.empty(self.topk, dtype=torch.int32, device=dev)
        wts = torch.empty(self.topk, device=dev)
        sg = torch.empty(1, device=dev)
        counter = torch.zeros(4, dtype=torch.int32, device=dev)
        act = torch.empty((self.topk + 1) * self.I, device=dev)
        for L in self.layers:
            self.lib.dr_router_topk(P(L["router"]), P(x), P(L["nw"]), self.eps, P(logits), self.E, self.topk, self.H,
                                    P(idx), P(wts), P(sg), P(counter), None, None, None, None, 0, 0, 0, 0, st)
            dec = self.lib.dr_moe_decode_fp8 if self.fp8 else self.lib.dr_moe_decode
            dec(P(L["gu_q"]), P(L["gu_s"]), P(L["d_q"]), P(L["d_s"]), P(L["sgu_q"]), P(L["sgu_s"]), P(L["sd_q"]),
                P(L["sd_s"]), P(x), P(idx), P(wts), P(sg), P(x), P(act), P(x), self.H, self.I, self.topk, P(L["nw"]),
                self.eps, None, 0, st)
