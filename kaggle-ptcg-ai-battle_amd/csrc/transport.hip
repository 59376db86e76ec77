// Rollout transport: pinned host mirrors of the env-side arrays, their HBM
// counterparts and one stream per env buffer — the reference's vecenv GPU
// mode (native/src/vecenv.h:498-545 allocation, :300-372 per-step copies).
//
// Per (buffer, time step) the reference runs: the policy forward + draw on
// the buffer's stream (net_callback), D2H of the buffer's actions, a checked
// stream sync, the env step on the host, then async H2D of the buffer's
// observations, rewards and terminals (and action mask) — the next step's
// forward is ordered after them on the same stream.  Here:
// ptcg_transport_step (captured rollout graph replay + download) and
// ptcg_transport_upload.  Buffers are contiguous agent slices
// [buf * apb, (buf + 1) * apb) of every array.  Buffer b's rollout graph runs
// on the trainer's rollout policy b (its own activations), so the buffers'
// forwards may overlap on their streams, as the reference's per-buffer
// threads do: ptcg_transport_launch queues a buffer's forward, draw and
// action download without waiting, ptcg_transport_wait ends in its checked
// stream sync, and ptcg_transport_step is the two in a row.
#include <string.h>
#include <vector>

#include "model.h"
#include "../../include/ptcg_amd.h"

struct PtcgTransport {
    int total = 0, nbuf = 0, apb = 0, natn = 0, mask_bytes = 0;
    int64_t obs_floats = 0;
    int dev = 0;
    // host (pinned) and device arrays, indexed by PtcgTransportArray
    void* host[PTCG_TR_COUNT] = {};
    void* devp[PTCG_TR_COUNT] = {};
    size_t bytes[PTCG_TR_COUNT] = {};
    std::vector<hipStream_t> streams;
};

namespace {

// record the message, return the code (for paths that must release first)
#define PT_FAIL(code, ...) (ptcg_set_error(__VA_ARGS__), (code))

// bytes of one agent's entry in array `a`
size_t entry_bytes(const PtcgTransport* x, int a) {
    switch (a) {
        case PTCG_TR_OBS: return (size_t)x->obs_floats * sizeof(float);
        case PTCG_TR_ACTIONS: return (size_t)x->natn * sizeof(float);
        case PTCG_TR_MASK: return (size_t)x->mask_bytes;
        default: return sizeof(float);   // rewards, terminals, logprobs, values
    }
}

void release(PtcgTransport* x) {
    for (auto s : x->streams)
        if (s) (void)hipStreamDestroy(s);
    for (int a = 0; a < PTCG_TR_COUNT; ++a) {
        if (x->host[a]) (void)hipHostFree(x->host[a]);
        if (x->devp[a]) (void)hipFree(x->devp[a]);
    }
    delete x;
}

int copy_slice(PtcgTransport* x, int a, int buf, hipMemcpyKind kind) {
    if (!x->bytes[a]) return PTCG_OK;
    const size_t eb = entry_bytes(x, a), off = (size_t)buf * x->apb * eb, n = (size_t)x->apb * eb;
    char* h = (char*)x->host[a] + off;
    char* d = (char*)x->devp[a] + off;
    if (kind == hipMemcpyHostToDevice) PT_HIP(hipMemcpyAsync(d, h, n, kind, x->streams[buf]));
    else PT_HIP(hipMemcpyAsync(h, d, n, kind, x->streams[buf]));
    return PTCG_OK;
}

}  // namespace

extern "C" int ptcg_transport_create(int total_agents, int num_buffers, int64_t obs_floats, int num_atns,
                                     int mask_bytes, PtcgTransport** out) {
    PT_REQUIRE(out, "transport_create: null out");
    *out = nullptr;
    PT_REQUIRE(total_agents >= 1 && num_buffers >= 1 && total_agents % num_buffers == 0,
               "transport_create: %d agents do not split into %d buffers", total_agents, num_buffers);
    PT_REQUIRE(obs_floats >= 1 && num_atns >= 1 && mask_bytes >= 0, "transport_create: bad entry sizes");
    auto* x = new PtcgTransport();
    x->total = total_agents;
    x->nbuf = num_buffers;
    x->apb = total_agents / num_buffers;
    x->natn = num_atns;
    x->mask_bytes = mask_bytes;
    x->obs_floats = obs_floats;
    int r = PTCG_OK;
    if (hipGetDevice(&x->dev) != hipSuccess) r = PT_FAIL(PTCG_ERR_HIP, "transport_create: no current device");
    for (int a = 0; a < PTCG_TR_COUNT && r == PTCG_OK; ++a) {
        x->bytes[a] = (size_t)total_agents * entry_bytes(x, a);
        if (!x->bytes[a]) continue;
        // logprobs and values stay on the device (the reference's rollout
        // buffers); the env reads actions and writes the rest
        const bool mirrored = a != PTCG_TR_LOGPROBS && a != PTCG_TR_VALUES;
        if (mirrored) {
            if (hipHostMalloc(&x->host[a], x->bytes[a], hipHostMallocPortable) != hipSuccess) {
                x->host[a] = nullptr;
                r = PT_FAIL(PTCG_ERR_HIP, "transport_create: pinned allocation of %zu bytes failed", x->bytes[a]);
                break;
            }
            memset(x->host[a], 0, x->bytes[a]);
        }
        if (hipMalloc(&x->devp[a], x->bytes[a]) != hipSuccess) {
            x->devp[a] = nullptr;
            r = PT_FAIL(PTCG_ERR_HIP, "transport_create: device allocation of %zu bytes failed", x->bytes[a]);
            break;
        }
        if (hipMemset(x->devp[a], 0, x->bytes[a]) != hipSuccess)
            r = PT_FAIL(PTCG_ERR_HIP, "transport_create: memset failed");
    }
    x->streams.assign(num_buffers, nullptr);
    for (int b = 0; b < num_buffers && r == PTCG_OK; ++b)
        if (hipStreamCreateWithFlags(&x->streams[b], hipStreamNonBlocking) != hipSuccess)
            r = PT_FAIL(PTCG_ERR_HIP, "transport_create: stream creation failed");
    if (r != PTCG_OK) {
        release(x);
        return r;
    }
    *out = x;
    return PTCG_OK;
}

extern "C" int ptcg_transport_free(PtcgTransport* x) {
    if (!x) return PTCG_OK;
    for (auto s : x->streams)
        if (s) (void)hipStreamSynchronize(s);
    release(x);
    return PTCG_OK;
}

extern "C" void* ptcg_transport_host(PtcgTransport* x, int which) {
    return x && which >= 0 && which < PTCG_TR_COUNT ? x->host[which] : nullptr;
}

extern "C" void* ptcg_transport_device(PtcgTransport* x, int which) {
    return x && which >= 0 && which < PTCG_TR_COUNT ? x->devp[which] : nullptr;
}

extern "C" void* ptcg_transport_stream(PtcgTransport* x, int buf) {
    return x && buf >= 0 && buf < x->nbuf ? (void*)x->streams[buf] : nullptr;
}

extern "C" int ptcg_transport_agents_per_buffer(PtcgTransport* x) { return x ? x->apb : 0; }

extern "C" int ptcg_transport_upload(PtcgTransport* x, int buf) {
    PT_REQUIRE(x && buf >= 0 && buf < x->nbuf, "transport_upload: buffer %d out of range", buf);
    PT_TRY(copy_slice(x, PTCG_TR_OBS, buf, hipMemcpyHostToDevice));
    PT_TRY(copy_slice(x, PTCG_TR_REWARDS, buf, hipMemcpyHostToDevice));
    PT_TRY(copy_slice(x, PTCG_TR_TERMINALS, buf, hipMemcpyHostToDevice));
    PT_TRY(copy_slice(x, PTCG_TR_MASK, buf, hipMemcpyHostToDevice));
    return PTCG_OK;
}

extern "C" int ptcg_transport_download(PtcgTransport* x, int buf) {
    PT_REQUIRE(x && buf >= 0 && buf < x->nbuf, "transport_download: buffer %d out of range", buf);
    PT_TRY(copy_slice(x, PTCG_TR_ACTIONS, buf, hipMemcpyDeviceToHost));
    // a failed sync leaves the env stepping on stale actions: report it
    const hipError_t e = hipStreamSynchronize(x->streams[buf]);
    if (e != hipSuccess) return PT_FAIL(PTCG_ERR_HIP, "transport_download: buffer %d stream sync: %s", buf,
                                        hipGetErrorString(e));
    return PTCG_OK;
}

extern "C" int ptcg_transport_capture_rollout(PtcgTransport* x, PtcgTrainer* t, int buf, int slot, uint64_t seed,
                                              uint64_t* step_dev) {
    PT_REQUIRE(x && t && buf >= 0 && buf < x->nbuf, "transport_capture_rollout: buffer %d out of range", buf);
    PT_REQUIRE(x->natn == 1, "transport_capture_rollout: the sampler draws one action per agent (num_atns %d)",
               x->natn);
    const int64_t row = ptcg_trainer_obs_size(t);
    PT_REQUIRE(row == x->obs_floats, "transport_capture_rollout: observation rows of %lld floats, trainer expects %lld",
               (long long)x->obs_floats, (long long)row);
    const size_t a0 = (size_t)buf * x->apb;
    return ptcg_trainer_capture_rollout_on(t, buf, slot, (const float*)x->devp[PTCG_TR_OBS] + a0 * x->obs_floats,
                                           nullptr, x->apb, seed, step_dev, (float*)x->devp[PTCG_TR_ACTIONS] + a0,
                                           (float*)x->devp[PTCG_TR_LOGPROBS] + a0,
                                           (float*)x->devp[PTCG_TR_VALUES] + a0);
}

extern "C" int ptcg_transport_launch(PtcgTransport* x, PtcgTrainer* t, int buf, int slot) {
    PT_REQUIRE(x && t && buf >= 0 && buf < x->nbuf, "transport_launch: buffer %d out of range", buf);
    PT_TRY(ptcg_trainer_replay_rollout(t, slot, x->streams[buf]));
    return copy_slice(x, PTCG_TR_ACTIONS, buf, hipMemcpyDeviceToHost);
}

extern "C" int ptcg_transport_wait(PtcgTransport* x, int buf) {
    PT_REQUIRE(x && buf >= 0 && buf < x->nbuf, "transport_wait: buffer %d out of range", buf);
    // a failed sync leaves the env stepping on stale actions: report it
    const hipError_t e = hipStreamSynchronize(x->streams[buf]);
    if (e != hipSuccess) return PT_FAIL(PTCG_ERR_HIP, "transport_wait: buffer %d stream sync: %s", buf,
                                        hipGetErrorString(e));
    return PTCG_OK;
}

extern "C" int ptcg_transport_step(PtcgTransport* x, PtcgTrainer* t, int buf, int slot) {
    PT_TRY(ptcg_transport_launch(x, t, buf, slot));
    return ptcg_transport_wait(x, buf);
}
