// lbh_cache.h — what the MoE entry points need from the HBM expert cache
// (lbh_cache.hip): the shape of its entries and the planes of a live lease.
#pragma once
#include <hip/hip_runtime.h>

#include "../../include/lightbridge_hip.h"
#include "lbh_internal.h"

namespace lbh {

struct CacheShape {
    ExpertDev views;   // gate / up / down views of an entry with null planes (the routed shape)
    uint32_t hidden, ffn;
    int32_t type_gate_up, type_down;
    int device;
};

bool cache_shape(const lbh_expert_cache *c, CacheShape *out);

// Planes of a live lease's entry and the event recorded after its upload;
// false when the lease is not live (released, or not from this cache).
bool cache_lease_planes(lbh_expert_cache *c, const lbh_expert_lease *lease, const uint8_t *planes[3],
                        hipEvent_t *ready);

// Records, on `stream`, that the work enqueued there so far reads the lease's
// slot: an upload that later refills the slot waits for it.  Call after
// enqueueing the readers and before releasing the lease.
bool cache_note_use(lbh_expert_cache *c, const lbh_expert_lease *lease, hipStream_t stream);

}  // namespace lbh
