"""The backend's C++ adapter (alphazero-go_amd/host/: HipBatchRunner,
makeHipRunner, HipInference, hip_probe) driven through the REFERENCE's own
InferenceHub, Network, self-play and arena code, compiled from the
reference's sources (with the `hip` name sites of oracle/hip_names.patch)
together with tests/hub_hip_driver.cpp (oracle/Makefile, target hubdriver).
This is the drop-in proof: the reference's unchanged hub batches many
workers' leaf requests into passes of this backend, and its unchanged
self-play and arena play the same games, byte for byte, whatever the
workers, pass caps and hub chaos.

Scenarios (tests/test_cuda.cpp:1022-1237, tests/test_inference_hub.cpp:272-628):
chaos batching with 16 workers (every row bit-identical to the position
alone; logits within maxErr 1e-5 and values within 1e-4 of Network::infer),
injected failure reaching every later
request, the memory refusal, argument refusals, the destructor draining
a delayed pass whose outputs are on the host when done comes, and the
ownership head through HipInference against the reference's own
Network::infer (naive backend) on a network with the head; and the
reference bench's hub load (256 threads of batch-8 requests, apps/bench.cpp:
282-307), whose positions per second it prints. The name sites:
checkBackendAvailable / cpuBackendName / makeBackend / the config's backend
key and WorkerEvaluators(net, "hip", ...) (tests/test_cuda.cpp:1240-1258).
The engine-spec sites: selfplay_engines / arena_engines naming hip engines
round-trip (tests/test_config.cpp:764-780), the hosts file's hip_workers sets
a hip engine's workers as cuda_workers does (tests/test_distributed.cpp:
347-349, 411-421), the engine fingerprint ends with the GPU description, and
the hub groups the coordinator's preflight checks are refused when they do
not fit.
Self-play slices on 5x5 and 9x9 networks and an arena wave of three networks
and a bot, byte-identical across workers {1, 3, 8}, pass caps {8, 256} and
chaos {off, on}, and the wave's slices joined equal to the whole
(tests/test_cuda.cpp:1270-1348).
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DRIVER = os.path.join(ROOT, "oracle", "_ref", "hub_hip_driver")

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("scenario", ["chaos", "failure", "memory", "refusals", "drain", "ownership", "throughput",
                                      "names", "engines", "selfplay", "arena"])
def test_reference_hub_drives_hip_runner(hip, scenario):
    # The driver is built beside the library (make -C oracle, from the
    # reference's sources): a library without it is an incomplete build, not
    # a reason to skip the drop-in proof.
    assert os.path.exists(DRIVER), f"{DRIVER} missing: build it with `make -C oracle hubdriver`"
    r = subprocess.run([DRIVER, scenario], capture_output=True, text=True, timeout=240)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert f"PASS {scenario}" in r.stdout
