"""The networks the engine evaluates and the CUDA-graph lanes that serve them, as the reference's engine/inference.py
builds them: answer_rows, FP16_RESIDUAL_SCALE, fp16_model and int8_model (:19-23, 238-278), and the graph lanes with
their lean answer rows (Lane, GraphedBatches, ImmediateBatches, serve and the graph sizes, :25-235). A lean lane's
answers are gathered on the GPU by chess_lean_answers, straight from the move logits and the expected scores, and its
launch and collect call the HIP runtime by address through engine.hip_runtime, as the native round loop does.
"""
from __future__ import annotations

from collections.abc import Callable
from multiprocessing import connection
from pathlib import Path

import numpy as np
import torch
from torch import nn

from engine.hip_runtime import DEVICE_TO_HOST, HOST_TO_DEVICE, hip_runtime
from model.checkpoint import load_model
from model.encoding import NUM_MOVE_IDS, START_POSITION_TOKENS, TOKENS_PER_BOARD
from model.hip_kernels import check, library_for, pointer, stream_of
from model.model import expected_score

#scales the residual stream down so its channels stay below fp16's largest number, 65,504
FP16_RESIDUAL_SCALE = 1 / 16


#a row per board: the move logits, then the expected score
def answer_rows(outputs: tuple[torch.Tensor, torch.Tensor] | torch.Tensor) -> torch.Tensor:
    if isinstance(outputs, torch.Tensor):
        return outputs
    move_logits, value_logits = outputs
    return torch.cat([move_logits.float(), expected_score(value_logits).unsqueeze(1)], dim=1)


def fused_model(model: nn.Module) -> nn.Module:
    """An fp32 ChessTransformer (on the GPU) as the fp16 inference network: residual stream scaled by 1/16, all but the heads in fp16."""
    from model.fused_blocks import FusedTransformer
    return FusedTransformer(model.scale_residual_stream(FP16_RESIDUAL_SCALE).half_except_heads(torch.float16))


def fp16_model(checkpoint_path: Path) -> nn.Module:
    """The network in fp16 (f32 sums), the heads in fp32."""
    return fused_model(load_model(checkpoint_path, torch.device("cuda")))


def int8_model(checkpoint_path: Path, fp16_blocks: int, weights: dict | None = None) -> nn.Module:
    """fp16_model with every block in int8 but the last and the fp16_blocks whose int8 costs the policy most.
    weights: the rounded weights (engine/quantization.py) if already read, else rounded once per checkpoint."""
    from model.int8_blocks import quantize_blocks
    from engine.quantization import int8_weights
    if weights is None:
        weights = int8_weights(checkpoint_path, fp16_blocks)
    return quantize_blocks(fp16_model(checkpoint_path), weights, FP16_RESIDUAL_SCALE)


def int8_network(model: nn.Module, weights: dict) -> nn.Module:
    """int8_model for a model already in memory (fp32, on the GPU): the benchmark's and the tests' random-init networks."""
    from model.int8_blocks import quantize_blocks
    return quantize_blocks(fused_model(model), weights, FP16_RESIDUAL_SCALE)


#answers a board: the move logits, then the expected score (reference engine/selfplay.py:46)
ANSWER_WIDTH = NUM_MOVE_IDS + 1
#a lean answer is the legal moves' logits in the search's order, padded with the expected score's index to
#LEGAL_SLOTS + 1 columns; a lean board row is the board's tokens, then those columns' int16 indices (the native crate's
#constants, reference engine/selfplay_rs/src/lib.rs:330-333, imported there from selfplay_rs)
LEGAL_SLOTS = 218
LEAN_COLUMNS = LEGAL_SLOTS + 1
LEAN_ROW = TOKENS_PER_BOARD + 2 * LEAN_COLUMNS


@torch.library.custom_op("chess::lean_answers", mutates_args=())
def lean_answers(answers: torch.Tensor, rows: torch.Tensor, columns_at: int, columns: int) -> torch.Tensor:
    """out[b][j] = answers[b] (a board's answer row: the move logits, then the expected score) at the int16 index stored at
    byte columns_at + 2j of rows[b]: reference Lane.answer's torch.gather (engine/inference.py:134-137) as one launch."""
    if answers.dtype != torch.float32 or rows.dtype != torch.uint8:
        raise ValueError(f"lean_answers takes f32 answer rows and uint8 board rows, not {answers.dtype} and {rows.dtype}")
    if answers.dim() != 2 or rows.dim() != 2 or rows.shape[0] != answers.shape[0]:
        raise ValueError(f"lean_answers: answer rows {tuple(answers.shape)}, board rows {tuple(rows.shape)}")
    library = library_for(answers.device)
    answers, rows = answers.contiguous(), rows.contiguous()
    out = torch.empty(answers.shape[0], columns, device=answers.device, dtype=torch.float32)
    code = library.chess_lean_answers(pointer(answers), pointer(rows), pointer(out), answers.shape[0], answers.shape[1], rows.shape[1], columns_at,
                                      columns, stream_of(answers.device))
    check(code, "lean_answers")
    return out


@lean_answers.register_fake
def _(answers, rows, columns_at, columns):
    return answers.new_empty(answers.shape[0], columns)


#a lean lane's answers for boards whose rows (tokens, then LEAN_COLUMNS int16 indices) are rows
def lean_rows(outputs: tuple[torch.Tensor, torch.Tensor] | torch.Tensor, rows: torch.Tensor) -> torch.Tensor:
    return lean_answers(answer_rows(outputs), rows, TOKENS_PER_BOARD, LEAN_COLUMNS)


#the L2 a position's activations take between a block's kernels, per unit of the model's width (reference :25-32)
L2_BYTES_PER_POSITION_WIDTH = 1024
MIN_CHUNK_POSITIONS = 64


def chunk_positions(width: int, lanes: int) -> int:
    l2_bytes = torch.cuda.get_device_properties(torch.cuda.current_device()).L2_cache_size
    return max(MIN_CHUNK_POSITIONS, l2_bytes // (lanes * width * L2_BYTES_PER_POSITION_WIDTH) // 16 * 16)


def chunked_answer_rows(model: nn.Module, boards: torch.Tensor, chunk: int | None) -> torch.Tensor:
    parts = [answer_rows(model(part)) for part in boards.split(chunk or len(boards))]
    return parts[0] if len(parts) == 1 else torch.cat(parts)


def chunked_lean_rows(model: nn.Module, boards: torch.Tensor, rows: torch.Tensor, chunk: int | None) -> torch.Tensor:
    step = chunk or len(boards)
    parts = [lean_rows(model(part), part_rows) for part, part_rows in zip(boards.split(step), rows.split(step))]
    return parts[0] if len(parts) == 1 else torch.cat(parts)


def serve(network, boards: list[np.ndarray], answers: list[np.ndarray], connections: list, stop, served_calls, served_positions) -> None:
    """Answers the searches' requests (a count of boards in the slot's shared array) in batches, one batch on the GPU while
    the next gathers (reference :36-59)."""
    slot_of = {id(end): slot for slot, end in enumerate(connections)}

    def hand_out(requests: list[tuple[int, int]], launched) -> None:
        evaluated = network.collect(launched)
        offset = 0
        for slot, count in requests:
            answers[slot][:count] = evaluated[offset:offset + count]
            offset += count
            connections[slot].send(True)
        served_calls.value += 1
        served_positions.value += offset

    in_flight = None
    while not stop.is_set():
        #with a batch on the GPU, take only the requests already waiting, so that its answers wait for nothing more
        ready = connection.wait(connections, timeout=0 if in_flight else 0.1)
        requests = [(slot_of[id(end)], end.recv()) for end in ready]
        started = (requests, network.launch(np.concatenate([boards[slot][:count] for slot, count in requests]))) if requests else None
        if in_flight is not None:
            hand_out(*in_flight)
        in_flight = started


def small_graph_sizes(max_batch: int, chunk: int | None = None) -> list[int]:
    """Graph sizes 1 to max_batch: doubling to 16, then steps of a sixteenth (at least 4); past a chunk, whole chunks plus
    the same steps, so that no batch pads into a forward of its own (reference :61-69)."""
    chunk = min(chunk or max_batch, max_batch)
    steps = [1]
    while steps[-1] < chunk:
        steps.append(min(chunk, steps[-1] * 2 if steps[-1] < 16 else steps[-1] + max(4, steps[-1] // 16)))
    sizes = [whole + step for whole in range(0, max_batch, chunk) for step in steps]
    last = next(index for index, size in enumerate(sizes) if size >= max_batch)
    return sizes[:last + 1]


def graph_sizes(max_batch: int) -> list[int]:
    """64, then steps of 64 to 1024, of 128 to 2048 and of 256 past it, until max_batch is held (reference :71-75)."""
    sizes = [64]
    while sizes[-1] < max_batch:
        sizes.append(sizes[-1] + (64 if sizes[-1] < 1024 else 128 if sizes[-1] < 2048 else 256))
    return sizes


def clear_blas_workspaces() -> None:
    """Drops the BLAS library's workspaces, so that none made while a graph records lands in that graph's pool (reference
    :77-82); the heads' small layers run on it."""
    clear = getattr(torch._C, "_cuda_clearCublasWorkspaces", None)
    if clear is not None:
        clear()


clear_cublas_workspaces = clear_blas_workspaces


class Lane:
    """One batch in flight: a stream, a graph per size in a pool of its own, and the pinned buffers its boards and answers
    cross in (reference :84-143). A lean lane takes rows of LEAN_ROW bytes (tokens, then LEAN_COLUMNS int16 indices of
    the answer columns) and answers LEAN_COLUMNS floats a board. warm_up: the model runs once a size before recording."""

    def __init__(self, model: nn.Module, sizes: list[int], chunk: int | None, lean: bool = False, warm_up: bool = True):
        self.stream = torch.cuda.Stream()
        self.device = torch.cuda.current_device()
        #launched and not yet collected: another launch would write over its answers
        self.pending = False
        self.lean = lean
        largest = sizes[-1]
        #recorded on a real position
        self.boards = torch.tensor([START_POSITION_TOKENS], dtype=torch.long, device="cuda").repeat(largest, 1)
        if lean:
            self.rows = torch.zeros(largest, LEAN_ROW, dtype=torch.uint8, device="cuda")
            self.rows[:, :TOKENS_PER_BOARD] = self.boards
            #every column the expected score's until a launch fills the rows
            self.rows[:, TOKENS_PER_BOARD:].view(torch.int16).fill_(ANSWER_WIDTH - 1)
            self.rows_host = torch.zeros(largest, LEAN_ROW, dtype=torch.uint8, pin_memory=True)
            self.rows_array = self.rows_host.numpy()
        else:
            self.boards_host = torch.zeros(largest, TOKENS_PER_BOARD, dtype=torch.long, pin_memory=True)
            self.boards_array = self.boards_host.numpy()
        self.answers_host = torch.zeros(largest, LEAN_COLUMNS if lean else ANSWER_WIDTH, dtype=torch.float32, pin_memory=True)
        self.answers_array = self.answers_host.numpy()
        self.done = torch.cuda.Event(blocking=True)

        #a graph records after warm-up calls off the default stream
        self.stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(self.stream), torch.no_grad():
            for size in sizes if warm_up else []:
                self.answer(model, size, chunk)
        torch.cuda.current_stream().wait_stream(self.stream)

        #a pool a lane, so that two lanes' graphs never share activations
        self.pool = torch.cuda.graph_pool_handle()
        self.graphs, self.answers = {}, {}
        for size in reversed(sizes):
            self.graphs[size] = torch.cuda.CUDAGraph()
            clear_blas_workspaces()
            with torch.cuda.graph(self.graphs[size], pool=self.pool, stream=self.stream), torch.no_grad():
                self.answers[size] = self.answer(model, size, chunk)
            clear_blas_workspaces()
        #the event has a handle from its first record on
        self.done.record(self.stream)
        self.done.synchronize()
        #a lean collect copies the answers' bytes as they are
        assert not lean or all(answers.dtype == torch.float32 and answers.is_contiguous() for answers in self.answers.values())

    def answer(self, model: nn.Module, size: int, chunk: int | None) -> torch.Tensor:
        if not self.lean:
            return chunked_answer_rows(model, self.boards[:size], chunk)
        self.boards[:size].copy_(self.rows[:size, :TOKENS_PER_BOARD])
        return chunked_lean_rows(model, self.boards[:size], self.rows[:size], chunk)

    def handles(self) -> dict:
        """The raw handles a lean launch and collect pass to the HIP runtime; graphs maps a size to (its executable graph, its
        answers on the device)."""
        return {"device": self.device, "stream": self.stream.cuda_stream, "done": self.done.cuda_event,
                "rows_host": self.rows_host.data_ptr(), "rows": self.rows.data_ptr(), "answers_host": self.answers_host.data_ptr(),
                "graphs": {size: (graph.raw_cuda_graph_exec(), self.answers[size].data_ptr()) for size, graph in self.graphs.items()}}


class GraphedBatches:
    """The model as graphs in in_flight lanes (reference :145-226): launch returns at once and collect waits, in any
    order, with at most in_flight batches out. A batch takes the smallest graph that holds it, on the first free lane.
    chunk: boards a forward (chunk_positions; None: a batch's all at once). blocking_wait: collect sleeps until the batch
    is done rather than spinning a core. lean: lean lanes, filled by the caller (rows_array) and run by launch_filled."""

    def __init__(self, model: nn.Module, sizes: list[int], in_flight: int = 2, chunk: int | None = None,
                 blocking_wait: bool = False, lean: bool = False):
        #kept alive: the graphs read its weights where they were recorded
        self.model = model
        self.sizes = sizes
        self.lanes = [Lane(model, sizes, chunk, lean, warm_up=number == 0) for number in range(in_flight)]
        self.lean = lean
        self.blocking_wait = blocking_wait
        self.runtime = hip_runtime() if lean else None
        self.handles = {id(lane): lane.handles() for lane in self.lanes} if lean else {}

    def launch(self, boards: np.ndarray) -> tuple[Lane, int, int]:
        if self.lean:
            raise RuntimeError("lean lanes answer rows with their columns (launch_filled), not boards")
        lane = self.free_lane()
        lane.boards_host[:len(boards)] = torch.from_numpy(boards)
        return self.launch_filled(lane, len(boards))

    def free_lane(self) -> Lane:
        """The lane the next launch takes; a caller may fill its boards_array (a lean lane's rows_array) for launch_filled."""
        lane = next((lane for lane in self.lanes if not lane.pending), None)
        if lane is None:
            raise RuntimeError("more batches in flight than lanes")
        return lane

    def launch_filled(self, lane: Lane, count: int) -> tuple[Lane, int, int]:
        """Starts the lane's first count boards; a lean lane's calls leave the thread's current device at the lane's."""
        size = next((size for size in self.sizes if size >= count), None)
        if size is None:
            raise ValueError(f"{count} boards are more than the largest graph's {self.sizes[-1]}")
        if lane.lean:
            runtime, handles = self.runtime, self.handles[id(lane)]
            stream = handles["stream"]
            runtime.check(runtime.set_device(handles["device"]), "the lane's device")
            runtime.check(runtime.memcpy(handles["rows"], handles["rows_host"], count * LEAN_ROW, HOST_TO_DEVICE, stream), "the boards' copy")
            lane.pending = True
            runtime.check(runtime.graph_launch(handles["graphs"][size][0], stream), "the graph's launch")
            runtime.check(runtime.event_record(handles["done"], stream), "the batch's event")
            return lane, size, count
        lane.pending = True
        with torch.cuda.stream(lane.stream):
            lane.boards[:count].copy_(lane.boards_host[:count], non_blocking=True)
            lane.graphs[size].replay()
            if self.blocking_wait:
                lane.done.record(lane.stream)
        return lane, size, count

    def collect(self, launched: tuple[Lane, int, int]) -> np.ndarray:
        """The batch's answers in the lane's pinned buffer. Copied here, not at launch: the GPU's copies queue, so a copy at
        launch would hold the other lane's boards behind it."""
        lane, size, count = launched
        if lane.lean:
            runtime, handles = self.runtime, self.handles[id(lane)]
            stream = handles["stream"]
            runtime.check(runtime.set_device(handles["device"]), "the lane's device")
            if self.blocking_wait:
                runtime.check(runtime.event_synchronize(handles["done"]), "the batch")
            answers = handles["graphs"][size][1]
            runtime.check(runtime.memcpy(handles["answers_host"], answers, count * LEAN_COLUMNS * 4, DEVICE_TO_HOST, stream), "the answers' copy")
            runtime.check(runtime.stream_synchronize(stream), "the batch")
            lane.pending = False
            return lane.answers_array[:count]
        if self.blocking_wait:
            lane.done.synchronize()
        with torch.cuda.stream(lane.stream):
            lane.answers_host[:count].copy_(lane.answers[size][:count])
        lane.pending = False
        return lane.answers_host[:count].numpy()

    def rust_network(self) -> dict:
        """What the native round loop holds: the lean lanes' handles (it keeps this object, so every lane lives while it runs)."""
        if not self.lean:
            raise ValueError("the native round loop needs lean lanes")
        return {"blocking_wait": self.blocking_wait, "lanes": [self.handles[id(lane)] for lane in self.lanes]}

    def settle(self) -> None:
        for lane in self.lanes:
            if lane.pending:
                lane.stream.synchronize()
                lane.pending = False


class ImmediateBatches:
    """GraphedBatches' interface without a GPU: launch does the work (reference :228-235)."""

    def __init__(self, evaluate_boards: Callable[[np.ndarray], np.ndarray]):
        self.evaluate_boards = evaluate_boards

    def launch(self, boards: np.ndarray) -> np.ndarray:
        return self.evaluate_boards(boards)

    def collect(self, launched: np.ndarray) -> np.ndarray:
        return launched
