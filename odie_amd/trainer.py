"""One training step of the packed multi-expert model on the GPU.

This is the native step of the reference (Probe::step, odie/native/runtime.cu:246-312, for
the hash-grid representation with the router disabled), with the single hash grid replaced
by one hash grid per image tile:

  ids --route--> (perm, local xy, offsets, pixels)    odie_route (no reference counterpart)
      --encode forward--> raw fp16 [n, 32]            GridEncoding fwd       (:260)
      --decoder + loss + backward--> dz, dW           decoder fwd/bwd, loss  (:270-273, :53-63)
      --encode backward--> grid gradient (scale 128)  GridEncoding bwd       (:282-287)
      --Adam--> grid master + fp16 copy (scale 128), decoder master + fp16 copy (scale 16384)

With router=True the gate (odie_gate_forward / odie_gate_backward) scales each level's features
before the decoder and turns the decoder's input gradient into the grid's upstream.

With fused=True (the default) the grid's Adam step runs inside the encode backward
(odie_grid_backward_adam): the gradient never reaches memory, and self.gradient is unused.
Without the router, planes=True (the default) has the decoder write the grid's upstream in the
encode backward's own level-major layout with its 128-row maxima (odie_mlp_train_planes,
odie_grid_backward_adam_planes), so the backward does not transpose it; the result is the same,
bit for bit.  With it, handoff=True (the default) has the encode forward also fill what the
backward would otherwise form in passes of its own (its slice masks, or its band lists:
odie_grid_forward_handoff, odie_grid_backward_adam_planes_handoff); again bit for bit.

With slots (int32 [regions_y * regions_x], tile -> expert, -1: none; allocate_tiles forms it
from a predicate and a parameter budget) only `experts` tables exist: ids of tiles without an
expert are routed after every expert's (odie_route_allocated), read zero features and train only
the decoder, as the reference's cells off their supports do.

Every buffer is allocated once, at construction, for `batch` ids; a step allocates nothing
on the device beyond the library's grow-once workspace.
"""
import numpy as np
import torch

from . import _lib, synth
from .decoder import Decoder
from .experts import ExpertGrid, Routing, route
from .gate import Gate
from .optimizer import FusedAdam

GRID_SCALE, HEAD_SCALE = 128.0, 16384.0   # loss scales (odie/native/runtime.cu:59,305-308)


class ExpertTrainer:
    def __init__(self, image, encoding, regions_x, regions_y, batch, *, grid_lr=1e-2, decoder_lr=1e-3, seed=0,
                 device='cuda', fused=True, router=False, gate_lr=1e-3, coarse_levels=0, activation='sigmoid',
                 planes=True, slots=None, experts=None, handoff=True):
        if isinstance(image, torch.Tensor):    # already on the device (gigapixel images)
            if image.dtype != torch.uint8 or image.ndim != 3 or image.shape[2] != 3:
                raise ValueError('image must be uint8 [height, width, 3]')
            rgb = image.contiguous().reshape(-1).to(device)
        else:
            image = np.ascontiguousarray(image, dtype=np.uint8)
            if image.ndim != 3 or image.shape[2] != 3:
                raise ValueError('image must be uint8 [height, width, 3]')
            rgb = torch.from_numpy(image.reshape(-1)).to(device)
        self.height, self.width = image.shape[:2]
        self.regions = (regions_x, regions_y)
        self.batch = batch
        self.fused = fused          # grid Adam applied inside the encode backward
        tiles = regions_x * regions_y
        if slots is not None:
            slots = torch.as_tensor(slots, dtype=torch.int32)
            if slots.numel() != tiles or experts is None or not 1 <= experts < 4096:
                raise ValueError('slots must map every tile; experts within 1..4095')
            if experts == tiles and torch.equal(slots.cpu(), torch.arange(tiles, dtype=torch.int32)):
                slots = None   # every tile owns its own expert: the plain route, the same result
        if slots is None:
            experts, self.slots = tiles, None
        else:
            self.slots = slots.to(device).contiguous()
        self.experts = experts
        self.rgb = rgb
        self.grid = ExpertGrid(encoding, experts, dtype=torch.float16, device=device)
        total = self.grid.table.numel()
        # fp32 master, uniform(-1e-4, 1e-4) as TCNN's HashGrid initializes its tables
        self.master = torch.from_numpy(synth.table(seed, total)).to(device)
        self.grid.table.copy_(self.master)
        self.grid_optimizer = FusedAdam(self.master, grid_lr, variant='tcnn', half_copy=self.grid.table)
        self.decoder = Decoder(seed=seed, device=device)
        # router (odie/native/runtime.cu:266-269,276-282): the gate scales each level's features
        self.gate = Gate(seed=seed, coarse=coarse_levels, activation=activation, device=device) if router else None
        if router:
            self.gate_optimizer = FusedAdam(self.gate.params, gate_lr, variant='tcnn_dense', half_copy=self.gate.half)
            self.weighted = torch.empty((batch, 32), dtype=torch.float16, device=device)
            self.sigmoid = torch.empty((batch, 16), dtype=torch.float32, device=device)
            self.upstream = torch.empty((batch, 32), dtype=torch.float16, device=device)
        self.decoder_optimizer = FusedAdam(self.decoder.params, decoder_lr, variant='tcnn_dense',
                                           half_copy=self.decoder.half)
        self.routing = Routing(torch.empty(batch, dtype=torch.int32, device=device),
                               torch.empty((batch, 2), dtype=torch.float32, device=device),
                               torch.empty(experts + 1, dtype=torch.int32, device=device), None,
                               torch.empty(batch, dtype=torch.int32, device=device))
        need = _lib.library().odie_route_workspace(batch, experts + (self.slots is not None))
        if need < 0:
            raise ValueError('invalid batch size for routing')
        self.workspace = torch.empty(max(need, 4), dtype=torch.uint8, device=device)
        self.raw = torch.empty((batch, self.grid.width), dtype=torch.float16, device=device)
        self.dz = torch.empty((batch, self.grid.width), dtype=torch.float16, device=device)
        self.gradient = None if fused else torch.empty(total, dtype=torch.float32, device=device)
        self.squares = torch.empty(batch, dtype=torch.float32, device=device)
        self.planes = planes and fused and not router
        self.handoff = handoff and self.planes
        if self.planes:
            self.plane_buffer = torch.empty(16 * batch, dtype=torch.int32, device=device)
            self.max_buffer = torch.empty(32 * ((batch + 127) // 128), dtype=torch.float32, device=device)
        if self.handoff:
            self.handoff_buffer = torch.empty(max(self.grid.handoff_bytes(batch), 1), dtype=torch.uint8, device=device)
        if self.grid.width != 32:
            raise ValueError('the decoder takes 32 input features (16 levels x 2)')

    def step(self, ids, update=True, mark=None, uniforms=None):
        """Train on int64 pixel ids [n] (n <= batch); returns the squared errors fp32 [n] in
        routed order (entry j belongs to ids[self.routing.perm[j]]).  With ids None and
        uniforms fp32 [n, 2], the batch is the stratified draw on those uniforms, computed
        inside the route (the ids never reach memory; perm[j] is then a stratified slot).
        mark(name), if given, is called after each stage is queued (for stage timing)."""
        n = ids.numel() if ids is not None else uniforms.shape[0]
        if not 1 <= n <= self.batch:
            raise ValueError('batch size must be within 1..%d' % self.batch)
        mark = mark or (lambda name: None)
        r = self.routing
        view = Routing(r.perm[:n], r.coords[:n], r.offsets, None, r.colors[:n])
        # the route writes each slot's pixel index; the decoder reads the target's bytes itself
        route(ids, self.width, self.height, *self.regions, out=view, workspace=self.workspace, pixels=True,
              uniforms=uniforms, slots=self.slots, experts=self.experts if self.slots is not None else None)
        mark('route')
        # with the planes path the forward also fills the backward's handoff (sized per call: the
        # backward's plan follows the tuning)
        handoff = None
        if self.handoff and update:
            need = self.grid.handoff_bytes(n)
            if need > self.handoff_buffer.numel():
                self.handoff_buffer = torch.empty(need, dtype=torch.uint8, device=self.handoff_buffer.device)
            handoff = self.handoff_buffer[:need] if need > 0 else None
        raw = self.grid.forward(view.coords, view.offsets, out=self.raw[:n], handoff=handoff)
        mark('encode_forward')
        features = raw
        if self.gate is not None:
            features, sigmoid = self.gate.forward(raw, weighted=self.weighted[:n], sigmoid=self.sigmoid[:n])
        # squared errors stay in routed order (slot j is id perm[j]); their mean is the loss
        if self.planes and update:
            planes, blockmax = self.decoder.train_planes(
                features, n, pixels=view.colors, rgb=self.rgb, squares=self.squares[:n], planes=self.plane_buffer[:16 * n].view(16, n),
                blockmax=self.max_buffer[:32 * ((n + 127) // 128)].view(-1, 32))
            mark('decoder')
            self.grid.backward_adam_planes(view.coords, view.offsets, planes, blockmax, self.grid_optimizer,
                                           loss_scale=GRID_SCALE, handoff=handoff)
            mark('encode_backward')
            mark('grid_adam')
            self.decoder_optimizer.step(self.decoder.grad, loss_scale=HEAD_SCALE)
            mark('decoder_adam')
            return self.squares[:n]
        self.decoder.train(features, n, pixels=view.colors, rgb=self.rgb, squares=self.squares[:n], dz=self.dz[:n])
        upstream = self.dz[:n]
        if self.gate is not None:
            upstream = self.gate.backward(raw, self.dz[:n], sigmoid, upstream=self.upstream[:n])
        mark('decoder')
        if update and self.fused:
            self.grid.backward_adam(view.coords, view.offsets, upstream, self.grid_optimizer, loss_scale=GRID_SCALE)
            mark('encode_backward')
            mark('grid_adam')
        else:
            self.grid.backward(view.coords, view.offsets, upstream, gradient=self.gradient, accumulate=False)
            mark('encode_backward')
        if update:
            if not self.fused:
                self.grid_optimizer.step(self.gradient, loss_scale=GRID_SCALE)
                mark('grid_adam')
            self.decoder_optimizer.step(self.decoder.grad, loss_scale=HEAD_SCALE)
            if self.gate is not None:
                self.gate_optimizer.step(self.gate.grad, loss_scale=HEAD_SCALE)
            mark('decoder_adam')
        return self.squares[:n]
