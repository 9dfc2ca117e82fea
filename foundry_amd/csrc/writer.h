// writer.h -- the .cugraph v1 archive of one graph's JSON document (writer.cpp).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace fdy {

// Archive bytes into `out`; 0, or an FDY_E_* code with `error` set.
int cugraph_from_json(const char* text, size_t len, std::vector<uint8_t>& out, std::string& error);

// The key the LOAD path groups a graph read from its JSON document by: its
// topology_key if non-empty, else the key recomputed from its nodes
// (csrc/CUDAGraphParallel.cpp:1791-1841).
int load_topology_key(const char* text, size_t len, std::string& key, std::string& error);

// The archive the LOAD path restores a graph read from its JSON document
// from: cugraph_from_json's, with load_topology_key's key in its
// TOPOLOGY_KEY section.
int cugraph_for_load(const char* text, size_t len, std::vector<uint8_t>& out, std::string& error);

}  // namespace fdy
