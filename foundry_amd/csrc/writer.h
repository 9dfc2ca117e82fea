// writer.h -- the .cugraph v1 archive of one graph's JSON document (writer.cpp).
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace fdy {

// Archive bytes into `out`; 0, or an FDY_E_* code with `error` set.
int cugraph_from_json(const char* text, size_t len, std::vector<uint8_t>& out, std::string& error);

}  // namespace fdy
