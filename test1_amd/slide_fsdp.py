"""SlideFSDP: train a HuggingFace causal LM one unit at a time on one GPU.

Drop-in for reference slide_fsdp.py:116-744: ``SlideFSDP(model, config)``
is an ``nn.Module`` whose ``forward(input_ids, attention_mask, labels)``
runs the forward, runs the backward itself and returns
``CausalLMOutputWithPast``; the host LayerAdam updates every unit as soon as
its gradients are on the host, so callers never call ``optimizer.step()``.

The model is split into units ``[embedding] + decoder layers + [norm +
lm_head]`` (reference slide_fsdp.py:213-244).  fp32 masters of every unit
live in host memory (pinned, or pageable with bf16 H2D).  On the GPU a unit
is bf16, in one of the ``gpu_buffer_pool_size`` pool units, as in the
reference, or in a buffer of its own when HBM allows (``resident_layers``);
an own buffer keeps the forward's weights for the backward and is staged with
the next step's weights right after the unit's update.  Unit i+1 is loaded
while unit i computes (``PreLayerFunction``), a pool unit is released after
its forward (``PostLayerFunction``), and in backward each unit's gradients go
to the host and into LayerAdam while earlier units are still computing; the
update thread takes the units the next forward needs first.  The embedding
moves only the batch's rows (``row_sparse_embedding``).  Checkpoint inputs are
offloaded by ``SlidingCheckpoint``.

Single GPU only: ``param_transfer_mode="full"`` and no collectives (the
reference's ``NoOpSync``, distributed_sync.py:313-362).

Differences from the reference, each a correctness or memory fix:
  * a unit's gradients are offloaded when all of them have been accumulated
    (post-accumulate-grad hooks on every parameter), not from a pre-hook on
    its first parameter (slide_fsdp.py:419-430), which fires before the
    unit's backward has finished;
  * the last decoder's gradients are the ones autograd produced: the
    reference leaves its ``param.grad`` outside the unit grad buffer and then
    offloads a stale buffer (layer_state.py:286-287, 370-375);
  * a decoder layer returning a tensor (transformers >= 5) is not indexed
    with ``[0]``, which would drop all but the first sequence of the batch
    (slide_fsdp.py:584-590);
  * ``save_pretrained`` restores the fp32 masters after writing bf16 weights
    (slide_fsdp.py:721-725 leaves the parameters detached from them);
  * the mask slot of the activation offload is allocated only if a mask
    tensor is actually saved;
  * padding masks are built with transformers' ``create_causal_mask`` when
    the decoder has no ``_update_causal_mask`` (transformers >= 5), where the
    reference drops them (slide_fsdp.py:557-561).
The performance options (own buffers, staging after updates, update order,
row-sparse embedding, bf16 H2D, SDMA gradient copies) change no bits.
"""

from __future__ import annotations

import os
import warnings
from typing import List, Optional

import torch
import torch.nn as nn
from torch.utils.checkpoint import checkpoint
from transformers.modeling_outputs import CausalLMOutputWithPast

from . import _native, kernels
from .config import SlideFSDPConfig
from .distributed_sync import create_distributed_sync
from .fused_ce import chunked_linear_cross_entropy
from .layer_state import GradSlotRing, LayerRuntimeState, StreamingRuntime
from .optimizer import LayerAdam
from .sliding_checkpoint import ActivationRing, KeptOnDevice, SlidingCheckpoint, StorageSpill, pin_or_keep


try:  # transformers >= 5: masks are built by a module-level function
    from transformers.masking_utils import create_causal_mask as _hf_create_causal_mask
except ImportError:  # older versions keep the decoder's _update_causal_mask
    _hf_create_causal_mask = None

class OutputLayer(nn.Module):
    """Final norm + lm_head + shifted cross-entropy as one unit (reference
    slide_fsdp.py:45-113).  ``fused=False``: full logits and
    ``nn.CrossEntropyLoss``, the reference's branch without a fused kernel;
    ``fused=True``: the chunked linear + cross entropy of ``fused_ce`` in
    place of the reference's optional fused kernel (loss only, no logits,
    as that branch)."""

    def __init__(self, norm: nn.Module, lm_head: nn.Module, hidden_size: int, fused: bool = False,
                 chunk_rows: int = 0):
        super().__init__()
        self.norm = norm
        self.lm_head = lm_head
        self.hidden_size = hidden_size
        self.fused = fused
        self.chunk_rows = chunk_rows
        self.lce = chunked_linear_cross_entropy if fused else None
        self.loss_fn = nn.CrossEntropyLoss()

    def forward(self, hidden_states: torch.Tensor, labels: Optional[torch.Tensor] = None):
        hidden_states = self.norm(hidden_states)
        loss = None
        logits = None
        if labels is not None and self.fused:
            shift_hidden = hidden_states[..., :-1, :].contiguous().view(-1, self.hidden_size)
            shift_labels = labels[..., 1:].contiguous().view(-1)
            loss = self.lce(shift_hidden, self.lm_head.weight, shift_labels, self.loss_fn.ignore_index,
                            self.chunk_rows)
            return loss, logits
        logits = self.lm_head(hidden_states)
        if labels is not None:
            shift_logits = logits[..., :-1, :].contiguous()
            shift_labels = labels[..., 1:].contiguous()
            loss = self.loss_fn(shift_logits.view(-1, shift_logits.size(-1)), shift_labels.view(-1))
        return loss, logits


def _cpu_count() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def adam_threads() -> int:
    """Threads of the host AdamW: ``SF_ADAM_THREADS`` if set above 0, else the
    host's cores (capped by the outer level of ``OMP_NUM_THREADS``) minus one.  The core left over
    keeps the threads that feed the GPU (the training loop / autograd thread
    and the offload thread, which mostly wait) responsive while an update
    saturates the rest; the reference reserves cores the same way with
    numa_launch.sh:255-266.  Measured on a 16-core host, Llama-3-8B step,
    same box: 14 threads 810-830 ms, 15 threads 785-793 ms, 16 threads
    785-796 ms."""
    raw = os.environ.get("SF_ADAM_THREADS", "").strip()
    if raw:
        try:
            env = int(raw)
        except ValueError:
            env = -1
        if env < 0:
            raise ValueError(f"SF_ADAM_THREADS={raw!r}: expected a thread count (0: the default)")
        if env > 0:
            return env
    n = _cpu_count()
    # OpenMP allows a list per nesting level ("16,4"); the outer level counts
    omp = os.environ.get("OMP_NUM_THREADS", "").split(",")[0].strip()
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n - 1)


# Seconds a host wait of the runtime (a pool unit, a gradient slot, a unit's
# offload or update, a copy's completion) may take before it raises.
DEFAULT_WAIT_TIMEOUT = 600.0


class SlideFSDP(nn.Module):
    """Layer-streaming trainer (reference slide_fsdp.py:116-211).

    Extra keyword arguments (all optional, not in the reference):
      stage_chunk_elems  fp32 elements per H2D staging chunk (default: the
                         largest unit, i.e. one chunk per unit)
      stage_depth        staging ring depth (default 3: copies may run up to
                         two units ahead of the unit being cast)
      grad_ring_depth    pinned gradient slots of the largest unit's size, or
                         None (default): one slot per unit, sized to it, so
                         gradient offload never waits for the host optimizer
                         (2 bytes of pinned host memory per parameter)
      wait_timeout       seconds before a host wait raises TimeoutError
                         naming the unit (default 600: a lost copy
                         completion or a wedged worker thread ends the step
                         with an error instead of blocking it forever, as
                         the reference's unbounded waits would; None: wait
                         without limit)
      d2h_engine         "sdma" (default): gradient D2H on SDMA engines of its
                         own; "kernel": by a capped-grid pack kernel writing
                         into host memory (slows the backward kernels beside
                         it); "copy": hipMemcpyAsync per parameter
      h2d_format         "fp32" (default): the fp32 masters (pinned) cross the
                         host link and are cast to bf16 on the GPU; "bf16":
                         the host optimizer keeps a pinned bf16 copy of every
                         master (written in its update pass) and that crosses
                         the link, half the bytes, while the fp32 masters
                         stay in pageable memory.  Both stage the same bits.
      resident_layers    decoder layers (the last ones, besides the last
                         decoder, which always stays) given a device buffer
                         of their own: loaded once per step in the forward
                         and kept for the backward instead of reloaded.
                         Costs 2 bytes per parameter of HBM per layer.
                         None (default): as many as fit in half of the free
                         device memory; 0: reload every unit, as the
                         reference (slide_fsdp.py:443-444).
      row_sparse_embedding  True (default): the embedding unit moves only the
                         rows a batch uses (lookup rows gathered from the host
                         table, gradient rows offloaded); False: the whole
                         table both ways, as the reference.  Same bits.
      stage_after_update  True (default): a unit with its own device buffer
                         is staged with its updated weights by the update
                         thread right after its update, i.e. during the
                         backward, when the host-to-device direction of the
                         link is idle, instead of in the next forward.  With
                         every decoder resident, the last decoder and the
                         output unit get own buffers too.  Same bits.
      fused_cross_entropy  False (default): full logits + nn.CrossEntropyLoss,
                         the reference's path without its optional fused
                         kernel; True: chunked linear + cross entropy (loss
                         only, no [B,S,V] logits), in place of that kernel.
      update_piece_elems  elements per piece of a unit's update (default 0:
                         whole units; e.g. 2**26).  A unit's gradients come
                         back in pieces, the host AdamW starts on the first
                         piece to land, and each updated piece is copied to
                         the device while the next is updated (one cast per
                         unit after its last piece).  Same bits: a piece
                         boundary inside a parameter falls on a 16-element
                         boundary of the update's vector body.  Shortens the
                         chain from the last update of the forward to the
                         first of the backward (the host AdamW idles 23 ms
                         per Llama-3-8B step instead of 51), but where host
                         memory bandwidth bounds the step it does not raise
                         the rate (measured within noise on a 16-core host).
      early_embedding_update  True (default): with the row-sparse embedding,
                         the table rows a batch does not touch (zero
                         gradient) get their AdamW update as the backward
                         starts, while the host AdamW would otherwise wait
                         for the first gradients; the batch's rows follow
                         once their gradient has landed.  Same bits.
      checkpoint_d2h     how checkpoints reach their pinned host slots:
                         "sdma" (the default with d2h_engine="sdma"), an SDMA
                         engine started by a worker thread once the layer's
                         input is on the device; "kernel", a 16-workgroup
                         kernel on the D2H stream.  A kernel writing into host
                         memory slows the kernels beside it (a bf16 GEMM ran
                         24-27 % slower), an SDMA engine does not.  Same bits.
      h2d_issue_limit    3 (default; 0: no limit): the forward and the
                         backward wait before a unit's load while that many
                         unit copies are still queued on the H2D stream.  A
                         queued HIP copy holds an SDMA engine, and later
                         copies then land on engines 4-7, which copy slower:
                         in the 2-unit pool schedule up to eight engines were
                         held at once.  There (Llama-3.1-8B, alternating, two
                         boxes) 4,204-4,340 tokens/s against 4,200-4,246,
                         H2D 52.0-52.6 GB/s against 50.7-51.1 while busy;
                         units with their own buffers rarely load in the
                         forward, and the default step was unchanged.
      cast_at_use        True (default): with fp32 H2D, a unit's fp32 master
                         is copied into a device fp32 slot of its own size
                         (right after its update for a unit with its own
                         buffer, else when the unit is loaded), and its cast
                         to bf16 runs where the unit is next used, on the
                         forward's or the backward's stream right before its
                         kernels, with the HBM to itself.  False: the cast
                         runs on a stream of its own as soon as the copy has
                         landed, beside the GEMMs of the unit computing
                         meanwhile.  Same bits; costs up to 4 bytes of HBM
                         per parameter (at most a quarter of the device
                         memory, else the ring).
      bf16_reload        None (default: True with fp32 H2D and bf16 units):
                         a unit reloaded for its backward (no device buffer
                         of its own) comes back as bf16 from a pinned bf16
                         copy of its master, which its update writes in the
                         same pass, instead of as fp32 plus a cast: half the
                         host-link bytes of the backward's reloads.  Same
                         bits (the master does not change between a unit's
                         forward and its backward).  Costs 2 bytes per
                         parameter of pinned host memory for those units,
                         pinned after the gradient slots; units the host
                         cannot pin reload fp32.
    """

    def __init__(self, model, config: SlideFSDPConfig, *, stage_chunk_elems: Optional[int] = None,
                 stage_depth: int = 3, grad_ring_depth: Optional[int] = None,
                 wait_timeout: Optional[float] = DEFAULT_WAIT_TIMEOUT,
                 d2h_engine: str = "sdma", h2d_format: str = "fp32",
                 resident_layers: Optional[int] = None, row_sparse_embedding: bool = True,
                 fused_cross_entropy: bool = False, stage_after_update: bool = True,
                 update_piece_elems: int = 0, cast_at_use: bool = True, early_embedding_update: bool = True,
                 bf16_reload: Optional[bool] = None, checkpoint_d2h: Optional[str] = None,
                 h2d_issue_limit: int = 3):
        super().__init__()
        if config.param_transfer_mode != "full":
            raise NotImplementedError("SlideFSDP runs on one GPU: only param_transfer_mode='full' is supported")
        self.config = config
        self.device = torch.device(config.device)
        if self.device.type != "cuda":
            raise ValueError(f"SlideFSDP needs a GPU device, got {self.device}")
        self.dtype = config.dtype
        self.base_model = model
        self.model_config = model.config
        self.rank = 0
        self.world_size = 1
        self.dist_sync = create_distributed_sync(config)

        self._fused_ce = bool(fused_cross_entropy)
        self._split_model(model)
        self.max_param_size = self._calculate_max_param_size()
        self.total_params = sum(sum(p.numel() for p in layer.parameters()) for layer in self.all_layers)

        chunk = int(stage_chunk_elems) if stage_chunk_elems else self.max_param_size
        self.runtime = StreamingRuntime(self.device, self.dtype, self.max_param_size, config.gpu_buffer_pool_size,
                                        chunk, stage_depth, grad_ring_depth, wait_timeout, d2h_engine=d2h_engine,
                                        h2d_format=h2d_format)
        if update_piece_elems < 0:
            raise ValueError("update_piece_elems must be >= 0")
        self.runtime.piece_elems = int(update_piece_elems)
        if h2d_issue_limit < 0:
            raise ValueError("h2d_issue_limit must be >= 0")
        self.runtime.h2d_issue_limit = int(h2d_issue_limit)
        self.runtime.cast_at_use = bool(cast_at_use) and h2d_format == "fp32"
        self._early_embedding_update = bool(early_embedding_update)
        self.buffer_pool = self.runtime.pool
        self.layer_optimizer = self._create_optimizer(config)
        self.layer_states: List[LayerRuntimeState] = []
        self._create_layer_states()
        if row_sparse_embedding and self._row_sparse_ok():
            self.layer_states[0].enable_row_sparse()
        self.runtime.init_grad_slots({s.layer_idx: s.total_size for s in self.layer_states if not s.row_sparse})
        # Updates run in the order the next forward loads units: the first
        # decoder, then the embedding, then the rest.
        self.runtime.update_priority = lambda u: 1 - u if u <= 1 else u
        self.runtime.stage_after_update = bool(stage_after_update)
        self._make_resident(self._auto_resident() if resident_layers is None else int(resident_layers))
        if bf16_reload is None:
            bf16_reload = h2d_format == "fp32" and self.dtype == torch.bfloat16
        self.bf16_reload_units = self._enable_bf16_reloads() if bf16_reload else []
        if not config.enable_activation_checkpoint and not self._all_units_own_buffers():
            # Without checkpoints the backward reads the weights the forward
            # saved, so no unit may go back to the 2-unit pool in between
            # (the reference's pool would overwrite them: slide_fsdp.py:399-400
            # releases each unit after its forward).
            raise NotImplementedError(
                "enable_activation_checkpoint=False needs every decoder and the output unit in a device "
                "buffer of its own (resident_layers = decoders - 1 and room for the last two units); "
                "with fewer, a reused pool unit would overwrite weights saved for backward")
        self._setup_autograd_functions()

        # The recompute must replay the forward's random numbers only if a
        # decoder layer draws any (dropout in training); Llama-family layers
        # draw none, and then the checkpoint skips stashing the RNG state.
        self._layer_uses_rng = self._decoders_use_rng()
        self.layer_tensors: Optional[List[List[torch.Tensor]]] = None
        self.position_embeddings = None
        self._act_ring = ActivationRing(self.device, wait_timeout=wait_timeout)
        if checkpoint_d2h is None:
            checkpoint_d2h = "sdma" if d2h_engine == "sdma" else "kernel"
        if checkpoint_d2h not in ("sdma", "kernel"):
            raise ValueError("checkpoint_d2h must be 'sdma' or 'kernel'")
        self._checkpoint_d2h = checkpoint_d2h
        if checkpoint_d2h == "sdma" and d2h_engine != "sdma":
            kernels.dma_init(self.device)
            kernels.require_routing_off()
        self._spill: Optional[StorageSpill] = None
        self._ring_grown = False
        self._ring_grow_pending = False
        self._act_paths: Optional[List[List[str]]] = None
        if config.ac_offload_mode == "nvme":
            # Checkpoint inputs on local storage, one file per (layer, tensor)
            # under ac_offload_dir.  The reference passes no file_paths in this
            # mode (slide_fsdp.py:592-600), so its SlidingCheckpoint asserts;
            # here they are made, and no per-layer pinned slots are allocated.
            os.makedirs(config.ac_offload_dir, exist_ok=True)
            tag = f"{os.getpid()}-{id(self)}"
            self._act_paths = [[os.path.join(config.ac_offload_dir, f"act-{tag}-{i}-{c}.bin") for c in range(4)]
                               for i in range(self.num_decoder_layers)]
            self._spill = StorageSpill(n_slots=6)
        self._print_model_info()

    # ------------------------------------------------------------------
    def _split_model(self, model) -> None:
        decoder = model.get_decoder()
        if hasattr(decoder, "layers"):
            layers = decoder.layers
        elif hasattr(decoder, "block"):
            layers = decoder.block
        else:
            raise ValueError("Cannot find decoder layers in model")
        self.num_decoder_layers = len(layers)
        self.embed_tokens = model.get_input_embeddings()
        self.decoder_layers = nn.ModuleList(layers)
        self.rotary_emb = getattr(decoder, "rotary_emb", None)
        self._update_causal_mask = getattr(decoder, "_update_causal_mask", None)
        lm_head = model.get_output_embeddings()
        if lm_head is not None and lm_head.weight is self.embed_tokens.weight:
            raise NotImplementedError("tied input/output embeddings are not supported (one parameter in two units)")
        self.output_layer = OutputLayer(norm=decoder.norm, lm_head=lm_head, hidden_size=model.config.hidden_size,
                                        fused=getattr(self, "_fused_ce", False))
        self.all_layers = [self.embed_tokens] + list(self.decoder_layers) + [self.output_layer]

    def _decoders_use_rng(self) -> bool:
        cfg = self.model_config
        for key in ("attention_dropout", "hidden_dropout", "resid_pdrop", "attn_pdrop", "dropout"):
            if float(getattr(cfg, key, 0.0) or 0.0) > 0.0:
                return True
        return any(isinstance(m, nn.Dropout) and m.p > 0 for layer in self.decoder_layers for m in layer.modules())

    def _calculate_max_param_size(self) -> int:
        return max(sum(p.numel() for p in layer.parameters()) for layer in self.all_layers)

    def _create_optimizer(self, config: SlideFSDPConfig) -> LayerAdam:
        opt = LayerAdam(lr=config.lr, betas=config.adam_betas, eps=config.adam_eps,
                        weight_decay=config.weight_decay, bias_correction=config.bias_correction,
                        fp32_optimizer_state=True, num_layer=len(self.all_layers),
                        nvme_offload_fraction=config.optimizer_nvme_offload_fraction,
                        offload_dir=config.optimizer_offload_dir, prefetch=True)
        opt.cpu_adam.set_num_threads(adam_threads())
        self.runtime.adam_threads = adam_threads()
        self.runtime._adam_threads_set = self.runtime.adam_threads
        # Updates run in next-forward order as gradients land, not in the
        # reference's backward order: take each update's bias corrections as
        # the reference's order gives them.
        opt.reference_order = True
        return opt

    def _create_layer_states(self) -> None:
        n = len(self.all_layers)
        for idx, layer in enumerate(self.all_layers):
            self.layer_states.append(LayerRuntimeState(layer, idx, self.config, self.runtime, self.layer_optimizer,
                                                       is_last_layer=(idx == n - 1)))

    def _act_prefetch_stream(self) -> torch.cuda.Stream:
        """Stream of the backward's checkpoint prefetches: behind the weight
        copies on the H2D stream, unless those run during the backward
        (staging after updates); then the D2H stream, which the SDMA gradient
        offload leaves free in the backward."""
        rt = self.runtime
        if rt.stage_after_update and rt.d2h_engine == "sdma":
            return rt.d2h_stream
        return rt.h2d_stream

    def _row_sparse_ok(self) -> bool:
        """The row gathers round to bf16: float16 units stage the embedding
        whole, as the reference does."""
        emb = self.embed_tokens
        return (self.dtype == torch.bfloat16 and isinstance(emb, nn.Embedding) and emb.max_norm is None
                and not emb.scale_grad_by_freq
                and not emb.sparse and emb.weight.shape[1] % 16 == 0 and len(list(emb.parameters())) == 1)

    def _auto_resident(self) -> int:
        """Decoder layers whose weights fit in half of the free device memory."""
        n_dec = len(self.layer_states) - 2
        if n_dec < 2:
            return 0
        free, _ = torch.cuda.mem_get_info(self.device)
        budget = free // 2
        elem = torch.empty((), dtype=self.dtype).element_size()
        k = 0
        for unit_idx in range(n_dec - 1, 0, -1):  # from the second-to-last decoder down
            need = self.layer_states[unit_idx].total_size * elem
            if need > budget:
                break
            budget -= need
            k += 1
        return k

    def _make_resident(self, k: int) -> None:
        n_dec = len(self.layer_states) - 2
        if k < 0 or k > max(0, n_dec - 1):
            raise ValueError(f"resident_layers must be in [0, {max(0, n_dec - 1)}]")
        # decoder units n_dec - 1 - k .. n_dec - 1 (unit index = decoder + 1);
        # the last decoder (unit n_dec) stays loaded through the pool anyway
        for unit_idx in range(n_dec - k, n_dec):
            st = self.layer_states[unit_idx]
            st.make_resident(torch.empty(st.total_size, dtype=self.dtype, device=self.device))
        self.resident_layers = k
        if self.runtime.stage_after_update and n_dec >= 1 and k == n_dec - 1:
            # Every decoder but the last has its own buffer: give the last
            # decoder and the output unit theirs as well, so that all units are
            # staged right after their update (the pool is then unused).
            free, _ = torch.cuda.mem_get_info(self.device)
            elem = torch.empty((), dtype=self.dtype).element_size()
            extra = [self.layer_states[n_dec], self.layer_states[n_dec + 1]]
            if sum(st.total_size for st in extra) * elem < free // 4:
                for st in extra:
                    st.make_resident(torch.empty(st.total_size, dtype=self.dtype, device=self.device))

    def _enable_bf16_reloads(self, reserve_bytes: int = 2 << 30) -> List[int]:
        """Give every decoder the backward reloads (no device buffer of its
        own; the last decoder stays loaded) a pinned bf16 copy of its master,
        until the host cannot pin more.  ``reserve_bytes`` of pinned memory
        are held meanwhile, so that the buffers pinned later (checkpoint
        slots, embedding rows) still fit under the driver's limit.  Returns
        the units that got one."""
        from .pinned import pinned_empty

        n_dec = len(self.layer_states) - 2
        todo = [st for st in self.layer_states[1:n_dec] if not st.resident_across_steps]
        if not todo:
            return []
        try:
            reserve = pinned_empty(reserve_bytes, torch.uint8)
        except _native.NativeError as e:
            if e.status != _native.HIP_ERROR_OUT_OF_MEMORY:
                raise
            print("SlideFSDP: no pinned memory left for bf16 reload copies; units reload their fp32 masters",
                  flush=True)
            return []
        got = []
        try:
            for st in todo:
                if not st.enable_bf16_reload():
                    print(f"SlideFSDP: bf16 reload copies pinned for {len(got)} units; the host cannot pin more, "
                          f"the others reload their fp32 masters", flush=True)
                    break
                got.append(st.layer_idx)
        finally:
            del reserve
        return got

    def _all_units_own_buffers(self) -> bool:
        return all(st._own_unit is not None for st in self.layer_states[1:])

    # ------------------------------------------------------------------
    def _setup_autograd_functions(self) -> None:
        """Autograd functions around each unit (reference slide_fsdp.py:343-430).

        ``PreLayerFunction`` (forward: prefetch the next unit, make the compute
        stream wait for this one) and ``PostLayerFunction`` (forward: release
        the unit; backward: prefetch the previous unit) are not re-run by the
        checkpoint recompute.  Gradient offload is driven by post-accumulate
        hooks on every parameter: when the last gradient of a unit lands, the
        unit is offloaded.
        """
        sf = self

        class PreLayerFunction(torch.autograd.Function):
            @staticmethod
            def forward(ctx, hidden_states, layer_state, next_layer_state):
                ctx.set_materialize_grads(False)
                ctx.layer_state = layer_state
                if next_layer_state is not None:
                    is_output = next_layer_state.layer_idx == len(sf.layer_states) - 1
                    next_layer_state.to_device_async(is_backward=is_output)
                layer_state._post_called = False
                layer_state.wait_for_h2d()
                sf.runtime.compute_mark(True)
                return hidden_states

            @staticmethod
            def backward(ctx, grad_output):
                # The gradient has flowed past the unit's first operation: all
                # of its backward kernels, including those reading its
                # weights, are enqueued.
                sf.runtime.compute_mark(False)
                ctx.layer_state.mark_backward_compute_done()
                return grad_output, None, None

        class PostLayerFunction(torch.autograd.Function):
            @staticmethod
            def forward(ctx, hidden_states, layer_state, is_last_layer):
                ctx.layer_state = layer_state
                ctx.set_materialize_grads(False)
                sf.runtime.compute_mark(False)
                if not is_last_layer:
                    layer_state.to_offload_async(is_backward=False)
                return hidden_states

            @staticmethod
            def backward(ctx, grad_output):
                sf._on_pre_backward(ctx.layer_state)
                return grad_output, None, None

        class EmbeddingRows(torch.autograd.Function):
            """Row-sparse lookup of the embedding unit.  The weight is an input
            only so that the output requires grad; its gradient goes to the
            host as rows (``offload_rows``), never into ``weight.grad``."""

            @staticmethod
            def forward(ctx, ids, layer_state, weight):
                ctx.layer_state = layer_state
                ctx.save_for_backward(ids)
                return layer_state.gather_rows(ids)

            @staticmethod
            def backward(ctx, grad_out):
                (ids,) = ctx.saved_tensors
                ctx.layer_state.offload_rows(grad_out, ids)
                return None, None, None

        self._PreLayerFunction = PreLayerFunction
        self._PostLayerFunction = PostLayerFunction
        self._EmbeddingRows = EmbeddingRows

        self._hook_handles = []
        for idx, state in enumerate(self.layer_states):
            state._post_called = False
            for p in state._grad_params:
                self._hook_handles.append(p.register_post_accumulate_grad_hook(self._make_grad_hook(state, idx)))

    def _make_grad_hook(self, state: LayerRuntimeState, idx: int):
        def hook(param):
            with state._grad_lock:
                if not state._bwd_armed or state._post_called:
                    return
                state._grads_seen += 1
                done = state._grads_seen == len(state._grad_params)
            if done:
                self._on_post_backward(state, idx)
        return hook

    def _on_pre_backward(self, layer_state: LayerRuntimeState) -> None:
        """Before a unit's backward: prefetch the unit before it, then order
        the compute stream after this unit's load (reference slide_fsdp.py:432-448)."""
        idx = layer_state.layer_idx
        if idx == len(self.layer_states) - 1:
            # First backward node of the step: flush units that never received
            # all their gradients once the backward pass has finished.
            torch.autograd.Variable._execution_engine.queue_callback(self._finish_backward)
        with layer_state._grad_lock:
            layer_state._bwd_armed = True
            layer_state._grads_seen = 0
        if idx == 0:
            # the embedding has no PreLayerFunction; its only backward kernel
            # (the gradient scatter) reads no weights
            layer_state._bwd_compute_done = True
        if idx - 1 >= 0:
            self.layer_states[idx - 1].to_device_async(is_backward=True)
        layer_state.wait_for_h2d()
        self._record_weights("weights_start", layer_state)
        if idx > 0:   # the embedding's backward (a gradient scatter) is not timed
            self.runtime.compute_mark(True)

    def _record_weights(self, what: str, layer_state: LayerRuntimeState) -> None:
        """Test hook (``runtime.capture_served``): a checksum of the unit's
        device weights, taken on the compute stream (the sum of their 16-bit
        words)."""
        served = self.runtime.capture_served
        unit = layer_state._current_gpu_cache
        if served is None or unit is None:
            return
        served[(what, layer_state.layer_idx)] = unit["param"][:layer_state.total_size].view(torch.int16).sum(
            dtype=torch.int64)

    def _on_post_backward(self, layer_state: LayerRuntimeState, idx: int) -> None:
        """After a unit's last gradient: pack, offload and queue the update
        (reference slide_fsdp.py:450-464)."""
        with layer_state._grad_lock:
            if layer_state._post_called:
                return
            layer_state._post_called = True
            layer_state._bwd_armed = False
        self._record_weights("weights_end", layer_state)
        layer_state.to_offload_async(is_backward=True)

    def _finish_backward(self) -> None:
        for idx, state in enumerate(self.layer_states):
            if state._bwd_armed and state.is_resident():
                self._on_post_backward(state, idx)
            if state.is_resident() and state._grads_offloaded:
                state.mark_backward_compute_done()

    # ------------------------------------------------------------------
    def _allocate_activation_tensors(self, batch_size: int, seq_length: int, hidden_size: int) -> None:
        """Pinned host slot of the hidden-state checkpoint per decoder layer
        (reference slide_fsdp.py:466-505); the mask slot is created on demand.
        A slot the host cannot pin (the driver's pinned-memory limit) keeps
        that layer's checkpoint in device memory; the reference raises there."""
        if self.config.ac_offload_mode == "none":
            return
        self.layer_tensors = [
            [pin_or_keep((batch_size, seq_length, hidden_size), self.dtype)]
            for _ in range(self.num_decoder_layers)
        ]
        kept = sum(isinstance(t[0], KeptOnDevice) for t in self.layer_tensors)
        if kept:
            warnings.warn(f"{kept} of {self.num_decoder_layers} checkpoint slots could not be pinned; "
                          "those layers keep their checkpoints in device memory")

    @staticmethod
    def _first(out):
        return out[0] if isinstance(out, (tuple, list)) else out

    def forward(self, input_ids: torch.Tensor, attention_mask: Optional[torch.Tensor] = None,
                labels: Optional[torch.Tensor] = None, **kwargs) -> CausalLMOutputWithPast:
        """One training step (reference slide_fsdp.py:507-640)."""
        batch_size, seq_length = input_ids.shape
        self._prepare_host_buffers(batch_size, seq_length)
        self._act_ring.reset()

        embed_state = self.layer_states[0]
        next_state = self.layer_states[1] if len(self.layer_states) > 1 else None
        # The first decoder's master was updated before the embedding's (the
        # embedding is the last unit of the previous backward), so its load is
        # issued first and runs while the embedding's update finishes.  The
        # reference issues the embedding first (slide_fsdp.py:536-541).
        if next_state is not None:
            next_state.to_device_async(is_backward=False)
        embed_state._post_called = False
        if embed_state.row_sparse:
            ids = input_ids if input_ids.device == self.device else input_ids.to(self.device)
            hidden_states = self._EmbeddingRows.apply(ids, embed_state, self.embed_tokens.weight)
        else:
            embed_state.to_device_async(is_backward=False)
            embed_state.wait_for_h2d()
            hidden_states = embed_state.layer(input_ids)
        hidden_states = self._PostLayerFunction.apply(hidden_states, embed_state, False)

        cache_position = torch.arange(0, seq_length, device=hidden_states.device)
        causal_mask = None
        if self._update_causal_mask is not None:
            causal_mask = self._update_causal_mask(attention_mask, hidden_states, cache_position, None, None)
        elif attention_mask is not None and _hf_create_causal_mask is not None:
            # transformers >= 5 builds the mask with a module-level function;
            # the reference only looks for the decoder method (slide_fsdp.py:234,
            # 557-561) and so drops padding masks with these versions.
            causal_mask = _hf_create_causal_mask(config=self.model_config, inputs_embeds=hidden_states,
                                                 attention_mask=attention_mask, past_key_values=None,
                                                 position_ids=cache_position.unsqueeze(0))
        if self.rotary_emb is not None and (self.position_embeddings is None
                                            or self.position_embeddings[0].shape[-2] != seq_length):
            # Cached per sequence length.  The reference computes them once
            # (slide_fsdp.py:564-566), so a batch of another length would get
            # the first batch's cos/sin.
            self.position_embeddings = self.rotary_emb(hidden_states, cache_position.unsqueeze(0))

        num_decoder_states = len(self.layer_states) - 2
        trace = self.runtime.log if self.runtime.trace is not None else None
        for i in range(num_decoder_states):
            layer_state = self.layer_states[i + 1]
            is_last_decoder = i == num_decoder_states - 1
            next_state = self.layer_states[i + 2]
            hidden_states = self._PreLayerFunction.apply(hidden_states, layer_state, next_state)

            def _layer_forward(h, mask, pos, layer):
                return self._first(layer(h, attention_mask=mask, position_embeddings=pos,
                                         output_attentions=False, use_cache=False))

            ckpt_kw = dict(use_reentrant=False, preserve_rng_state=self._layer_uses_rng)
            if not self.config.enable_activation_checkpoint:
                # every unit keeps its own device buffer (checked at construction):
                # the activations stay in HBM and the backward recomputes nothing
                hidden_states = _layer_forward(hidden_states, causal_mask, self.position_embeddings,
                                               layer_state.layer)
            elif self.config.ac_offload_mode != "none":
                with SlidingCheckpoint(layer_idx=i + 1, layer_tensors=self.layer_tensors,
                                       gds_offload=self._spill is not None, file_paths=self._act_paths,
                                       spill=self._spill, is_last_layer=is_last_decoder,
                                       no_mask=attention_mask is None, device=str(self.device),
                                       prefetch_ring=self._act_ring, trace=trace,
                                       max_workgroups=self.runtime.d2h_workgroups,
                                       stream=self.runtime.d2h_stream,
                                       prefetch_stream=self._act_prefetch_stream(),
                                       pack_fence=self.runtime.stager.fence_after_casts,
                                       link_timing=self.runtime.link_timing,
                                       on_prefetch_ready=self._reopen_compute,
                                       before_pin=self._drain,
                                       served=self.runtime.capture_served,
                                       pack_engine=self._checkpoint_d2h):
                    hidden_states = checkpoint(_layer_forward, hidden_states, causal_mask, self.position_embeddings,
                                               layer_state.layer, **ckpt_kw)
            else:
                hidden_states = checkpoint(_layer_forward, hidden_states, causal_mask, self.position_embeddings,
                                           layer_state.layer, **ckpt_kw)
            hidden_states = self._PostLayerFunction.apply(hidden_states, layer_state, is_last_decoder)

        output_state = self.layer_states[-1]
        hidden_states = self._PreLayerFunction.apply(hidden_states, output_state, None)
        loss, logits = self.output_layer(hidden_states, labels)
        if loss is not None:
            loss = self._PostLayerFunction.apply(loss, output_state, True)
            if self._early_embedding_update and torch.is_grad_enabled() and loss.requires_grad:
                # the backward below reaches the lookup: the embedding's
                # gradient-free rows can be updated while it starts
                self.layer_states[0].start_early_update()
            try:
                loss.backward()
            except BaseException:
                self._after_failed_backward()
                raise
            if isinstance(self.runtime.grad_ring, GradSlotRing) and not self._ring_grown:
                self._ring_grow_pending = True
        return CausalLMOutputWithPast(loss=loss, logits=logits)

    def _prepare_host_buffers(self, batch_size: int, seq_length: int) -> None:
        """Before a step's first copy: widen the gradient slot ring once (after
        the first step), and pin the buffers sized by the batch (checkpoint
        slots, embedding row buffers) on the first step or for a new batch
        shape.  Pinned memory is allocated only after ``_drain``, with no copy
        into or out of pinned memory in flight: copies of a previous step, or
        of forwards without a backward, may still run, and pinning near the
        driver's limit while copies ran has left wrong results."""
        hidden_size = self.model_config.hidden_size
        if self._ring_grow_pending:
            self._ring_grow_pending = False
            self._drain()
            self._grow_grad_ring()
        act_alloc = (self.config.ac_offload_mode == "cpu" and self.config.enable_activation_checkpoint
                     and (self.layer_tensors is None
                          or self.layer_tensors[0][0].shape != (batch_size, seq_length, hidden_size)))
        embed_rows = (self.layer_states[0].row_sparse
                      and not self.layer_states[0].host_buffers_fit(batch_size * seq_length))
        if act_alloc or embed_rows:
            self._drain()
            if act_alloc:
                self._allocate_activation_tensors(batch_size, seq_length, hidden_size)
            if embed_rows:
                self.layer_states[0].alloc_host_buffers(batch_size * seq_length)

    def _after_failed_backward(self) -> None:
        """The backward raised part-way (a hook, an out-of-memory error, an
        interrupt): the units it finished were offloaded and their updates
        queued, the others never were.  Let the queued work finish, close the
        embedding's early update part (its late part will not come), give
        back every unit still on the device and drop gradients, so the next
        step starts from the masters as they are.  Errors here are secondary
        to the one being raised and are not reported."""
        for s in self.layer_states:
            try:
                s.wait_for_update()
            except Exception:
                pass
        try:
            if self.layer_states[0].row_sparse:
                self.layer_states[0].settle_orphaned_early()
        except Exception:
            pass
        for s in self.layer_states:
            with s._grad_lock:
                s._bwd_armed = False
                s._post_called = False
                s._grads_seen = 0
            s.release_device_unit()
            for p in s._params:
                p.grad = None

    def _reopen_compute(self) -> None:
        """With link timing on: a unit's backward compute starts once its
        checkpoint prefetch has arrived, not when the stream began to wait."""
        if self.runtime.link_timing is not None:
            self.runtime.compute_mark(True)

    def _drain(self) -> None:
        """Wait for every queued offload and update and for the device: no copy
        into or out of pinned host memory is in flight afterwards."""
        self.wait_for_updates()
        torch.cuda.synchronize(self.device)
        self._act_ring.drain_packs()
        if self._spill is not None:
            # checkpoint copies into bounce slots run on the spill's worker
            self._spill.flush()

    def _grow_grad_ring(self) -> None:
        """At the start of the second step, with nothing in flight (``_drain``)
        and the first step's checkpoint slots and embedding rows pinned: widen
        a gradient slot ring (the fallback when one slot per unit does not fit)
        as far as pinned memory allows, leaving 1 GiB.  Growing pins buffers
        until the driver refuses one; that is not done while copies into
        other pinned buffers are in flight.  In the Qwen2.5-14B-shaped step
        with fp32 masters (pinned memory at the driver's cap), growing right
        after the first backward had been issued left the last units of that
        backward with non-finite gradients in 2 of 7 runs; at the drained
        point, 0 of 3."""
        ring = self.runtime.grad_ring
        if self._ring_grown or not isinstance(ring, GradSlotRing):
            return
        self._ring_grown = True
        before = ring.depth
        ring.grow(max_depth=ring.n_small, headroom_bytes=1 << 30)
        print(f"SlideFSDP: gradient slot ring {before} -> {ring.depth} slots", flush=True)

    # ------------------------------------------------------------------
    def wait_for_updates(self) -> None:
        """Block until every queued host update has finished."""
        for s in self.layer_states:
            s.wait_for_update()

    def release_device_units(self) -> None:
        """Give back every unit still loaded on the device and point all
        parameters at their fp32 masters.  After a forward without a backward
        (evaluation), units with a buffer of their own, the last decoder and
        the output unit stay loaded, with ``param.data`` their bf16 device
        views; call this before writing the masters directly (e.g.
        ``model.load_state_dict``), then ``refresh_host_copies``."""
        self.wait_for_updates()
        if self.layer_states and self.layer_states[0].row_sparse:
            self.layer_states[0].settle_orphaned_early()
        for s in self.layer_states:
            s.release_device_unit()

    def refresh_host_copies(self) -> None:
        """After the masters were written outside the optimizer (a loaded
        checkpoint): drop the stagings made for the next forward, so every
        unit is staged from its new master, and with h2d_format='bf16'
        recompute every unit's bf16 host copy.  Masters may only be written
        while no unit is loaded (``release_device_units``, which this calls
        as well)."""
        self.release_device_units()
        for s in self.layer_states:
            s.refresh_host_copy()

    def update_learning_rate(self, new_lr: float) -> None:
        if self.layer_optimizer is not None:
            self.layer_optimizer.update_learning_rate(new_lr)

    def clip_grad_norm_(self, max_norm: float) -> torch.Tensor:
        """Reference slide_fsdp.py:651-681, including its behaviour: updates run
        as each unit's gradients arrive, so by the time this is called every
        ``param.grad`` has been released and the norm is taken over none."""
        self.wait_for_updates()
        total = 0.0
        for s in self.layer_states:
            for p in s.layer.parameters():
                if p.grad is not None:
                    total += p.grad.data.float().norm(2).item() ** 2
        total = total ** 0.5
        coef = max_norm / (total + 1e-6)
        if coef < 1:
            for s in self.layer_states:
                for p in s.layer.parameters():
                    if p.grad is not None:
                        p.grad.data.mul_(coef)
        return torch.tensor(total)

    def _print_model_info(self) -> None:
        opt_bytes = self.total_params * 4 * 2
        print(f"\n{'=' * 60}\nSlideFSDP Model Info\n{'=' * 60}")
        print(f"Model type: {getattr(self.model_config, 'model_type', '?')}")
        print(f"Num decoder layers: {self.num_decoder_layers}")
        print(f"Total parameters: {self.total_params:,}")
        print(f"Max layer param size: {self.max_param_size:,}")
        print(f"Param transfer mode: {self.config.param_transfer_mode}")
        print(f"Grad sync mode: {self.config.grad_sync_mode}")
        print(f"World size: {self.world_size}")
        print("Estimated CPU memory:")
        print(f"  - Parameters (FP32): {self.total_params * 4 / 1e9:.2f} GB")
        print(f"  - Optimizer states: {opt_bytes / 1e9:.2f} GB")
        print(f"  - Total: {(self.total_params * 4 + opt_bytes) / 1e9:.2f} GB")
        print(f"GPU buffer pool: {self.config.gpu_buffer_pool_size} units\n{'=' * 60}\n")

    def save_pretrained(self, output_dir: str) -> str:
        """Write the model with bf16 weights (reference slide_fsdp.py:705-733),
        then point the parameters back at their fp32 masters."""
        os.makedirs(output_dir, exist_ok=True)
        self.wait_for_updates()
        saved = []
        with torch.no_grad():
            for s in self.layer_states:
                for p in s.layer.parameters():
                    saved.append((p, p.data))
                    p.data = p.data.to(dtype=self.dtype)
        try:
            self.base_model.save_pretrained(output_dir)
        finally:
            for p, d in saved:
                p.data = d
        print(f"Model saved to {output_dir}")
        return output_dir

    def close(self) -> None:
        """Finish queued work, stop the worker threads and detach the
        gradient hooks from the model's parameters (which would otherwise keep
        this wrapper's host state alive)."""
        try:
            if self.layer_states and self.layer_states[0].row_sparse:
                self.layer_states[0].settle_orphaned_early()
            self.wait_for_updates()
            self._act_ring.close()
        finally:
            for h in getattr(self, "_hook_handles", []):
                h.remove()
            self._hook_handles = []
            self.runtime.shutdown()
            self.runtime.release_slots(self.layer_states)
            if self._spill is not None:
                self._spill.close()
                self._spill = None
            if self.layer_optimizer.offloader is not None:
                self.layer_optimizer.offloader.flush()
            self.dist_sync.cleanup()

    def __del__(self):
        rt = getattr(self, "runtime", None)
        if rt is not None:
            if rt.offload_executor is not None:
                rt.offload_executor.shutdown(wait=False)
            rt.update_executor.shutdown(wait=False)
