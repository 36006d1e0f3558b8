/*
 * apus_container.h — host-side index of the routed-expert slabs of an apus
 * model container (safetensors shards + model.safetensors.index.json).
 * Internal to the backend; the C ABI is in include/apus_hip.h.
 */
#ifndef APUS_CONTAINER_H
#define APUS_CONTAINER_H

#include <stdint.h>

#include <string>
#include <vector>

#include "../../include/apus_hip.h"

struct ApusHipContainer {
    std::string dir;                     /* directory holding the index and shards */
    std::vector<std::string> shards;     /* shard file names, first-use order */
    int n_layers = 0, n_mtp = 0, E = 0;
    uint64_t slab_bytes = 0;
    std::vector<ApusHipSlabRec> recs;    /* [n_layers * E], layer-major */
};

/* Build the index (the same rules as c/cache.h:1030-1110 and :431-509).
 * Returns nullptr and writes err on failure. */
ApusHipContainer *apus_container_index(const char *model_dir, int n_layers, int n_mtp, int E,
                                       std::string &err);

#endif
