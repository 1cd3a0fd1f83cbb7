/* vq_format.hpp — host-side reader of RQVQ containers, the C++ counterpart of
 * the reference's Rust crate tools/vq-format (Container::open, Stage::open,
 * f16). It validates headers and locates stage payloads; decoding and every
 * matvec run on the GPU. */
#pragma once

#include <stddef.h>
#include <stdint.h>

#include <string>
#include <vector>

namespace sparkmv {
namespace fmt {

/* Exact IEEE half -> single, subnormals included (lib.rs:50-72). */
float f16(uint16_t h);

struct StageView {
    int dim = 0, nc = 0, rows = 0, cols = 0, nbit = 0;
    bool v3 = false;
    size_t mrow = 0, prow = 0, bytes = 0;
    const uint8_t * base = nullptr;
};

struct ContainerView {
    int dim = 0, nc = 0, rows = 0, cols = 0, nbit = 0;
    bool v3 = false;
    uint64_t payload = 0;
    size_t stride = 0;           /* bytes per stage payload */
    std::vector<StageView> stages;
};

/* Stage::open (lib.rs:94-156): false with `err` set on a refusal. */
bool open_stage(const uint8_t * p, size_t len, StageView & st, std::string & err);
/* Container::open (lib.rs:240-306). */
bool open_container(const uint8_t * buf, size_t len, ContainerView & c, std::string & err);

}  // namespace fmt
}  // namespace sparkmv
