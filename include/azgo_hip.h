/*
 * azgo_hip.h: the C ABI of the MI355X (gfx950) inference backend for the
 * residual policy/value network of robominds/alphazero-go.
 *
 * This is the drop-in boundary. The reference's GPU plug-in point is the
 * BatchRunner interface behind its InferenceHub
 * (include/azgo/inference_hub.hpp:41-53); its CUDA backend implements it in
 * src/cuda/cuda_runner.cu and exposes the rest through include/azgo/cuda.hpp.
 * Every entry point below replaces one of those, cited per function. The
 * thin C++ adapter that a maintainer adds to the reference tree (a
 * HipBatchRunner deriving from azgo::BatchRunner, makeHipRunner, ...) calls
 * only these functions.
 *
 * Conventions: plain pointers and sizes, no exceptions across the ABI. Every
 * function returning int returns AZH_OK (0) on success or a negative
 * AZH_ERR_* code, and then azh_last_error() (per thread) says what failed,
 * in the reference's wording where it has one ("hip: ...", "lower
 * inference_batch"). Arrays are fp32, row-major, the reference's layouts:
 * input [B][2H+2][n*n] (Evaluator::evaluate, include/azgo/evaluator.hpp:24),
 * logits [B][n*n+1], values [B] (tanh).
 */
#ifndef AZGO_HIP_H
#define AZGO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    AZH_OK = 0,
    AZH_ERR_ARGUMENT = -1,    /* std::invalid_argument in the reference */
    AZH_ERR_UNAVAILABLE = -2, /* no usable GPU / wrong architecture */
    AZH_ERR_MEMORY = -3,      /* std::runtime_error "... lower inference_batch" */
    AZH_ERR_TENSOR = -4,      /* std::logic_error naming a tensor (upload contract) */
    AZH_ERR_HIP = -5,         /* a HIP runtime error ("hip: ...") */
    AZH_ERR_STATE = -6,       /* a call the runner's state does not allow */
    AZH_ERR_FORMAT = -7       /* a checkpoint file loadNetwork would refuse (std::runtime_error naming the file) */
};

/* NetConfig (include/azgo/network.hpp:24-36). With ownership set the pass
 * also runs the ownership head (1x1 conv, BN, tanh per point,
 * src/network.cpp:298-308) and the network's tensors include it. */
typedef struct azh_netcfg {
    int board;        /* n: 5, 9, 13 or 19 */
    int history;      /* H: planes = 2H + 2 */
    int blocks;       /* residual blocks */
    int filters;      /* F */
    int value_hidden; /* V, at most 256 */
    int ownership;    /* 1: the network has the ownership head */
} azh_netcfg;

/* One named tensor of Network::params() / buffers() (src/network.cpp:113-165),
 * e.g. "block3.conv2.w", "policy.bn.runVar". */
typedef struct azh_tensor {
    const char* name;
    const float* data;
    size_t size; /* floats */
} azh_tensor;

typedef struct azh_runner azh_runner;

/* BatchRunner::begin's done callback (include/azgo/inference_hub.hpp:47-50):
 * called exactly once per pass, from the runner's completion thread, with
 * error NULL on success or a message ("hip: ..."). It must only mark and
 * wake (it may not call back into the runner). */
typedef void (*azh_done_fn)(void* user, int slot, const char* error);

/* ---------------------------------------------------------------- probes */

/* cudaBuilt (include/azgo/cuda.hpp:29-30): 1 in this library. */
int azh_built(void);

/* cudaAvailable (include/azgo/cuda.hpp:32-39; src/cuda/cuda_context.cu:32-87):
 * 1 when a gfx950 device is present and a first kernel ran; else 0 and, when
 * why is not NULL, the reason (e.g. "kernels built for gfx950; this GPU is
 * gfx942"). The first call sets up the process-wide HIP context. */
int azh_available(char* why, size_t cap);

/* cudaDescription (include/azgo/cuda.hpp:41-49): GPU name, gfx arch, HIP
 * runtime version and a hash of the kernel sources and flags. */
int azh_describe(char* out, size_t cap);

/* No counterpart in the reference: the compute units of the runner's device
 * (the current one), as the launch rules count them: a pass alone runs its
 * stem and tower as one board-resident launch when its batch gives one
 * workgroup to 95% of them or fills whole rounds of them, and a pass splits
 * into two half-batch chains by how its workgroups fill rounds of them.
 * AZH_ERR_UNAVAILABLE without a usable GPU. */
int azh_device_cus(int* cus);

/* The message of the calling thread's last failed call ("" if none). */
const char* azh_last_error(void);

/* ---------------------------------------------------------------- runners */

/* checkCudaInferenceMemory / hubBytes (include/azgo/cuda.hpp:60-66;
 * src/cuda/cuda_runner.cu:186-223): device bytes one runner of `slots` slots
 * of max_batch positions needs (weights included). */
int azh_memory_need(const azh_netcfg* cfg, int max_batch, int slots, size_t* bytes);

/* The same check the constructor makes: AZH_ERR_MEMORY with the reference's
 * message unless `hubs` runners of that shape fit in free memory less
 * 512 MB (or the test hook's limit). */
int azh_check_memory(const azh_netcfg* cfg, int max_batch, int hubs, int slots_per_hub);

/* GpuHubs (include/azgo/gpu_memory.hpp): `hubs` runners of `slots_per_hub`
 * slots of up to max_batch positions each. */
typedef struct azh_hub_group {
    int hubs;
    int slots_per_hub;
    int max_batch;
} azh_hub_group;

/* checkCudaInferenceMemory's overload over groups of hubs
 * (include/azgo/cuda.hpp:63-66; src/cuda/cuda_runner.cu:242-256): every
 * group's runners summed, against free memory less 512 MB. The refusal
 * names the total hub count and the largest max_batch. No group, or a
 * group with a count below 1, is AZH_ERR_ARGUMENT. */
int azh_check_memory_groups(const azh_netcfg* cfg, const azh_hub_group* groups, int count);

/* makeCudaRunner (include/azgo/cuda.hpp:53-58; src/cuda/cuda_runner.cu:227-234)
 * and CudaWeights::upload (src/cuda/cuda_network.cu:71-106): checks memory,
 * uploads the tensors once (the caller's arrays are not kept), allocates
 * `slots` (1..2) slots of max_batch positions, each with its own stream,
 * device workspace and pinned staging, and starts the completion thread.
 * The tensors must be exactly the network's params() and buffers(): an
 * unknown name, a wrong size, a missing tensor or a tensor this pass never
 * reads fail with AZH_ERR_TENSOR naming it. */
int azh_create(const azh_netcfg* cfg, const azh_tensor* tensors, int count, int max_batch, int slots,
               azh_runner** out);

/* Network::params() then Network::buffers() for cfg (src/network.cpp:113-165):
 * the number of tensors, and tensor i's name and size in floats. These are
 * the tensors azh_create takes and the order a checkpoint stores them in. */
int azh_tensor_count(const azh_netcfg* cfg, int* count);
int azh_tensor_info(const azh_netcfg* cfg, int i, char* name, size_t cap, size_t* size);

/* readCheckpointConfig (include/azgo/checkpoint.hpp:22; src/checkpoint.cpp:37-60,
 * 126-128): the network shape in an .azn checkpoint's header. Failures are
 * AZH_ERR_FORMAT with loadNetwork's message ("cannot open checkpoint <path>",
 * "<path>: not an AZGO checkpoint", "<path>: unsupported version 3",
 * "<path>: invalid network shape in header", "<path>: truncated", ...). */
int azh_checkpoint_config(const char* path, azh_netcfg* cfg);

/* loadNetwork (include/azgo/checkpoint.hpp:18-21; src/checkpoint.cpp:102-124)
 * into caller memory: the header into cfg and *floats = the total size of
 * every tensor; with values non-NULL (cap >= *floats) also every tensor,
 * concatenated in params() then buffers() order (azh_tensor_info), each
 * checked by position, name and size as loadNetwork checks it ("<path>:
 * tensor 3 is 'x' but expected 'y'", "has 7 tensors but the network needs
 * 9", "unexpected data after the last tensor", ...). */
int azh_checkpoint_read(const char* path, azh_netcfg* cfg, float* values, size_t cap, size_t* floats);

/* loadNetwork followed by makeCudaRunner: a runner straight from an .azn
 * checkpoint (file errors as azh_checkpoint_read, then azh_create's). */
int azh_create_from_checkpoint(const char* path, int max_batch, int slots, azh_runner** out);

/* Waits for every pass in flight, then frees everything
 * (CudaBatchRunner::~CudaBatchRunner, src/cuda/cuda_runner.cu:64-71). */
void azh_destroy(azh_runner* r);

int azh_slots(const azh_runner* r);     /* BatchRunner::slots */
int azh_max_batch(const azh_runner* r); /* BatchRunner::maxBatch */

/* BatchRunner::input / logits / values (include/azgo/inference_hub.hpp:46-52):
 * the slot's pinned host staging, [max_batch][planes][area],
 * [max_batch][area+1], [max_batch]. Outputs are valid after done until the
 * slot's next begin. NULL for a bad slot. */
float* azh_slot_input(azh_runner* r, int slot);
const float* azh_slot_logits(const azh_runner* r, int slot);
const float* azh_slot_values(const azh_runner* r, int slot);

/* BatchRunner::begin (include/azgo/inference_hub.hpp:47-50;
 * CudaBatchRunner::begin, src/cuda/cuda_runner.cu:79-105): enqueues copy
 * in, the pass on the first B positions of the slot's input, copy out and
 * an event, and returns at once; done(user, slot, error) follows from the
 * completion thread once the outputs are on the host. A B outside
 * [1, max_batch] or a busy slot fails here, before anything is enqueued
 * (the hub turns that into a failed batch). */
int azh_begin(azh_runner* r, int slot, int B, azh_done_fn done, void* user);

/* CudaInference::infer (include/azgo/cuda.hpp:68-84;
 * src/cuda/cuda_network.cu:314-339): the whole pass synchronously on slot
 * 0's resources; the slot must be idle. ownership [B][area] (after tanh) may
 * be NULL; non-NULL for a network without the head is AZH_ERR_ARGUMENT, as
 * CudaInference refuses it. */
int azh_infer(azh_runner* r, const float* input, int B, float* logits, float* values, float* ownership);

/* No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). azh_infer's pass on device arrays, enqueued on `stream`
 * (a hipStream_t; NULL: the null stream) without waiting and without
 * allocating: input [B][planes][area], logits [B][area+1], values [B] and,
 * when not NULL, ownership [B][area] (the network must have the head) are
 * the caller's device memory; the pass's own intermediates go to a static
 * 96 MiB device array per GPU, held until the process ends (256 boards of a
 * 19x19 network of 128 filters fit). A batch that needs more is
 * AZH_ERR_ARGUMENT, naming the most positions one call takes. Every call on
 * a GPU shares that GPU's array: calls that overlap on one GPU (two streams,
 * two threads) race and must be ordered by the caller. Nothing in the
 * array needs to start at zero (every element a pass reads is written
 * earlier in the same pass). The runner's device must be current; no slot
 * is used, so slots' passes may run meanwhile. Same kernels, same bits as
 * azh_infer. The call takes the launch forms of a pass alone when no slot
 * has a pass in flight; it is not itself counted as one (it may be captured
 * into a graph and replayed, so the library cannot tell when it runs), so a
 * slot's pass begun while it runs may take the forms of a pass alone too:
 * the same bits, only the two passes' speed differs. Safe under stream
 * capture (global mode): nothing on its path allocates or synchronizes. */
int azh_infer_noalloc(azh_runner* r, const float* input, int B, float* logits, float* values, float* ownership,
                      void* stream);

/* The legal-move softmax on the GPU (no reference counterpart on the GPU; it
 * restates Mcts::expand's priors, src/mcts.cpp:170-183): priors[b][a] =
 * exp(l - max) / sum over legal of the same, 0 where legal[b][a] == 0.
 * Host arrays [B][actions]; runs on its own stream and waits. */
int azh_softmax_legal(const float* logits, const uint8_t* legal, int B, int actions, float* priors);

/* ---------------------------------------------------------------- the steps either side of the pass */

/* encodePlanes (src/encode.cpp:14-43; include/azgo/encode.hpp:20-27) on the
 * GPU for B positions: stones [B][H][n*n] Color bytes (0 Empty, 1 Black,
 * 2 White; ply k = the position k moves ago, k = 0 the current one, as
 * Mcts::evaluateLeaves gathers them, src/mcts.cpp:119-132), plies[b] of them
 * present (1..H; NULL: all H), to_move[b] (1 Black, 2 White: "own" stones
 * are the side to move's), sym[b] (0..7, transformPoint; NULL: identity) ->
 * planes [B][2H+2][n*n]. Host arrays; waits. */
int azh_encode_planes(const uint8_t* stones, const int32_t* plies, const uint8_t* to_move, const uint8_t* sym, int B,
                      int n, int H, float* planes);

/* The legal actions Mcts::expand builds for a node (src/mcts.cpp:152-169) on
 * the GPU for B positions: Board::isLegal (src/board.cpp:131-150: empty,
 * not suicide) and positional superko: the stones after the move
 * (Board::hashAfter, src/board.cpp:176-190) may not hash to any of
 * seen[seen_offsets[b] .. seen_offsets[b+1]) (the game's positions and the
 * node's path, Zobrist hashes as Board::hash). stones [B][n*n], to_move[B]
 * (1 Black, 2 White) -> legal [B][n*n+1] (1 legal, 0 not; pass always 1).
 * Host arrays; waits. */
int azh_legal_moves(const uint8_t* stones, int n, const uint8_t* to_move, const uint64_t* seen,
                    const int64_t* seen_offsets, int B, uint8_t* legal);

/* A batch of positions as MCTS leaves hand them over: the arrays of
 * azh_encode_planes (stones [B][H][n*n] with ply 0 the board the legal
 * moves are for) and of azh_legal_moves (the superko lists). */
typedef struct azh_positions {
    const uint8_t* stones;       /* [B][H][n*n] */
    const int32_t* plies;        /* [B], 1..H; NULL: all H */
    const uint8_t* to_move;      /* [B], 1 Black, 2 White */
    const uint8_t* sym;          /* [B], 0..7; NULL: identity */
    const uint64_t* seen;        /* every position's superko hashes, concatenated */
    const int64_t* seen_offsets; /* [B+1] */
} azh_positions;

/* The leaf evaluation of Mcts::evaluateLeaves and the priors of
 * Mcts::expand (src/mcts.cpp:113-183) as one synchronous GPU call on slot
 * 0: positions encoded on the GPU, the pass, the legal actions, the logits
 * mapped back from each position's symmetry (action a <- logit
 * transformAction(sym, a), src/mcts.cpp:136-146), the softmax over the legal
 * actions. Outputs [B][n*n+1]: logits (mapped back; may be NULL), priors
 * (0 where illegal), legal; values [B]. The host copies carry stone bytes,
 * not planes: 2H+2 floats per point become H bytes. */
int azh_evaluate_positions(azh_runner* r, const azh_positions* pos, int B, float* logits, float* priors,
                           uint8_t* legal, float* values);

/* azh_evaluate_positions as an asynchronous pass on a slot, as azh_begin
 * runs azh_infer's (the positions path of Mcts::evaluateLeaves and
 * Mcts::expand, src/mcts.cpp:113-183, behind the hub's BatchRunner::begin,
 * src/inference_hub.cpp:222-227): the arrays of `pos` are checked, copied
 * into the slot's pinned staging (H stone bytes per point, not 2H+2 input
 * floats) and the call returns once the copies and kernels are enqueued;
 * done(user, slot, error) follows from the completion thread once the
 * outputs are in the slot's pinned buffers: azh_slot_position_logits,
 * azh_slot_priors, azh_slot_legal ([B][n*n+1] each) and azh_slot_values
 * ([B]), valid until the slot's next begin. Bad positions (as
 * azh_evaluate_positions checks them), a B outside [1, max_batch] or a
 * busy slot fail here, before anything is enqueued. Same kernels, same bits
 * as azh_evaluate_positions. The slot's positions buffers (device and
 * pinned) are allocated on its first positions call. */
int azh_begin_positions(azh_runner* r, int slot, int B, const azh_positions* pos, azh_done_fn done, void* user);
/* The outputs of the slot's last azh_begin_positions (NULL before its first):
 * logits mapped back from each position's symmetry, priors, legal. The
 * positions form of BatchRunner::logits (include/azgo/inference_hub.hpp:46-52),
 * carrying what Mcts::expand builds from the logits (src/mcts.cpp:152-183). */
const float* azh_slot_position_logits(const azh_runner* r, int slot);
const float* azh_slot_priors(const azh_runner* r, int slot);
const uint8_t* azh_slot_legal(const azh_runner* r, int slot);

/* HIP events on slot 0's stream around `iters` device-resident runs of each
 * step of azh_evaluate_positions, on positions staged once: ms[0] the
 * encoding, ms[1] the legal moves, ms[2] the priors, ms[3] the whole chain
 * (encoding, pass, legal moves, priors). Totals in milliseconds. */
int azh_time_positions(azh_runner* r, const azh_positions* pos, int B, int iters, float* ms);

/* Whether passes replay a captured hipGraph per batch size (default 1), or
 * launch their kernels one by one. Read when a pass is enqueued: set it
 * while no other thread is beginning a pass. */
int azh_set_graphs(azh_runner* r, int enabled);

/* Whether a small board's pass (5x5 up to 64 channels; 9x9 up to 32
 * channels, and up to 64 past 128 boards; 13x13 up to 16 channels, and up
 * to 32 past 100 boards) runs as one launch (stem, residual tower and
 * heads), one workgroup per board with the activations in LDS (default 1),
 * or as one launch per layer. Both give the same bits. Read when a pass is
 * enqueued: set it while no other thread is beginning a pass. No
 * counterpart in the reference (its CUDA runner launches per layer); a test
 * hook. */
int azh_set_small_tower(azh_runner* r, int enabled);

/* Whether a 19x19 pass of a 113-128 channel network runs its stem and
 * residual tower as one launch with each board resident in one workgroup
 * from the first layer to the last: 0 never (one launch per layer), 1 for a
 * pass enqueued while no other is in flight whose batch gives one
 * workgroup to at least 95% of the CUs, or to every CU in each of two or
 * more rounds (default), 2 at every batch. All give the same bits. Read when a pass is enqueued: set it while
 * no other thread is beginning a pass. No counterpart in the reference (its
 * CUDA runner launches per layer); a test hook. */
int azh_set_resident_tower(azh_runner* r, int mode);

/* ---------------------------------------------------------------- device-resident passes (measurement) */

/* Copies the first B positions of the slot's pinned input to its device
 * buffer and waits. */
int azh_stage(azh_runner* r, int slot, int B);
/* Enqueues the pass on the slot's stream over the staged device input, no
 * host copies (what a timed region measures with the inputs already in HBM). */
int azh_enqueue(azh_runner* r, int slot, int B);
/* Waits for the slot's stream. */
int azh_synchronize(azh_runner* r, int slot);
/* Copies the slot's device outputs for B positions into its pinned outputs and waits. */
int azh_fetch(azh_runner* r, int slot, int B);
/* HIP events on the slot's stream around `iters` device-resident passes:
 * total milliseconds. */
int azh_time_passes(azh_runner* r, int slot, int B, int iters, float* ms);
/* HIP events on the slot's stream around `iters` runs of the residual
 * tower as per-layer launches over the whole batch on one stream (every
 * block's two convolutions, in order, on the slot's staged data): total
 * ms, the number of launches timed and the number of layers they ran, for
 * the per-layer convolution's average launch time. */
int azh_time_tower_convs(azh_runner* r, int slot, int B, int iters, float* ms, int* launches, int* layers);

/* HIP events on the slot's stream around `iters` board-resident launches
 * over B boards (azh_set_resident_tower), with the stem first when `stem`
 * is nonzero (as a pass runs it) or the tower alone on the slot's staged
 * trunk: total ms. Refused for a network the resident tower does not take
 * (19x19, 113-128 channels, up to 32 input planes). */
int azh_time_resident_tower(azh_runner* r, int slot, int B, int iters, int stem, float* ms);

/* How a pass of B boards runs, as enqueued alone on the device (alone
 * nonzero) or beside another pass in flight: a mask of 1 (the small-board
 * pass in one launch), 2 (the stem and the tower board-resident in one
 * launch) and 4 (two half-batch chains on the slot's two streams); 0: one
 * launch per layer on one stream. */
int azh_pass_form(azh_runner* r, int B, int alone, int* form);

/* HIP events on the slot's stream around `iters` runs of the residual
 * tower as the pass runs it: one stream, or for a large batch two
 * half-batch chains on the slot's two streams, forked from and joined back
 * into its stream. Total ms and the number of layers (of the whole batch)
 * run: the tower's effective time per layer within a pass. */
int azh_time_tower_layers(azh_runner* r, int slot, int B, int iters, float* ms, int* layers);

/* Events around `iters` synchronous round trips: pinned H2D, pass, D2H. */
int azh_time_round_trips(azh_runner* r, int slot, int B, int iters, float* ms);

/* The runner kept full, as the reference's bench measures its GPU runner
 * (measureGpuPipelined, apps/bench.cpp:227-279): every slot always has a
 * pass of B in flight through azh_begin (pinned H2D, pass, D2H, the
 * completion thread's done), each slot resubmitted as soon as its done
 * comes, until `passes` passes have completed. Each slot's input must hold
 * B positions; every slot must be idle. *ms = wall milliseconds from the
 * first begin to the last done. A pass that fails stops the resubmission;
 * the passes in flight are drained and the error is returned. */
int azh_time_pipelined(azh_runner* r, int B, int passes, float* ms);

/* azh_time_pipelined for the positions path (measureGpuPipelined's loop,
 * apps/bench.cpp:227-279): every slot kept full through azh_begin_positions
 * on the same positions `pos` (B of them; host copies of stone bytes in,
 * logits, priors, legal actions and values out). */
int azh_time_pipelined_positions(azh_runner* r, const azh_positions* pos, int B, int passes, float* ms);

/* ---------------------------------------------------------------- kernel probes (tests) */

/* The pass's 3x3 convolution kernel alone (cuda_probe::convBnRelu,
 * include/azgo/cuda.hpp:123-126): x [B][cin][n*n], w [cout][cin*9],
 * y [B][cout][n*n] = relu?(scale*conv + shift (+ skip)). skip may be NULL.
 * tiling: -1 the pass's rule (for a pass alone on the device), else an index
 * 0..12 forcing a workgroup shape,
 * (16-channel blocks per wave, waves along channels, waves along the board's
 * 16-point column groups, groups per wave; 0 = all): 0 (2,2,2,12),
 * 1 (1,4,1,0), 2 (1,2,1,0), 3 (1,1,1,0), 4 (1,8,1,0), 5 (1,2,2,12),
 * 6 (1,1,4,6), 7 (1,1,4,2), 8 (1,1,4,1), 9 (1,1,8,1), 10 (1,1,3,1),
 * 11 (1,1,6,1), 12 (1,1,6,2). */
int azh_probe_conv3x3(const float* x, const float* w, const float* scale, const float* shift, const float* skip,
                      int relu, int B, int n, int cin, int cout, int tiling, float* y);

/* HIP events around `iters` launches of the 3x3 convolution kernel alone on
 * device-resident synthetic data (x [B][cin][n*n] -> y), tiling as above:
 * total ms. For tuning the workgroup shape. */
int azh_time_conv3x3(int B, int n, int cin, int cout, int tiling, int iters, float* ms);

/* The heads kernels alone on the runner's weights: trunk [B][F][n*n] ->
 * logits, values, and ownership [B][n*n] when non-NULL (the network must
 * have the head). */
int azh_probe_heads(azh_runner* r, const float* trunk, int B, float* logits, float* values, float* ownership);

/* The stem and the first `blocks` residual blocks on the runner's weights:
 * input [B][planes][n*n] -> trunk [B][F][n*n]. */
int azh_probe_trunk(azh_runner* r, const float* input, int B, int blocks, float* trunk);

/* cuda_probe::fill (include/azgo/cuda.hpp:101-103): data[0..n) = value on the
 * GPU; all n + tail floats travel, so a test can see the tail untouched. */
int azh_probe_fill(float* data, size_t n, float value, size_t tail);

/* A plain device-to-device copy of `bytes` (known traffic, to scale HBM
 * counters), repeated `iters` times; total ms. */
int azh_probe_copy(size_t bytes, int iters, float* ms);

/* The fp32 matrix units' rate with nothing else in the way (the measured
 * ceiling beside the published peak): one workgroup of 8 waves per CU, each
 * wave a dependent chain of 4 * chain v_mfma_f32_16x16x4_f32, launched
 * `iters` times; total ms and the flops of one launch. */
int azh_probe_mfma(int chain, int iters, float* ms, double* flops);

/* ---------------------------------------------------------------- test hooks (cuda_probe, include/azgo/cuda.hpp:138-155) */

/* Hub chaos seed WorkerEvaluators reads (cuda_probe::setHubChaosSeed). */
void azh_set_hub_chaos_seed(uint64_t seed);
uint64_t azh_hub_chaos_seed(void);
/* After n more passes complete normally the next one reports a failure
 * through done (once); 0 disables (cuda_probe::failPassesAfter). */
void azh_fail_passes_after(int n);
/* A stand-in for free device memory in the memory checks; 0 restores the
 * device's (cuda_probe::setMemoryLimit). */
void azh_set_memory_limit(size_t bytes);
/* Passes the runners of this process have reported (cuda_probe::passesCompleted). */
long long azh_passes_completed(void);
/* Holds each pass's stream this long before its copy-out
 * (cuda_probe::setCopyOutDelay). */
void azh_set_copy_out_delay(int microseconds);

#ifdef __cplusplus
}
#endif

#endif /* AZGO_HIP_H */
