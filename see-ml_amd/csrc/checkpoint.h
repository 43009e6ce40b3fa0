// checkpoint.h — the SEKP checkpoint container, host side (no GPU code).
//
// runtime/custodian/checkpoint.{h,cc}: a checkpoint is the arena's
// persistent segment (LoRA adapters + optimizer moments) plus the 1-indexed
// training step, bound to the plan that laid the segment out. Layout
// (little-endian, 40-byte header, version 3):
//   u32 magic "SEKP"; u32 version; u64 plan_hash; u64 step;
//   u64 persistent_size; u64 payload_hash (ContentHash64 of the payload);
//   payload (persistent_size bytes).
// Writes are durable: a temporary file is written, flushed to disk and
// renamed over the target, then the directory entry is flushed. Reads prove
// magic, version, plan binding, size and payload hash before any byte is
// handed out. Errors read "Checkpoint: <message>" with the reference's texts.
#pragma once

#include <cstdint>
#include <string>

#include "plan_checks.h"

namespace seeml_hip {

inline constexpr const char* kUnitCheckpoint = "Checkpoint";
inline constexpr uint32_t kCheckpointMagic = 0x504B4553;  // "SEKP"
inline constexpr uint32_t kCheckpointVersion = 3;

Status WriteCheckpoint(const std::string& path, uint64_t plan_hash, uint64_t step,
                       const uint8_t* payload, uint64_t size);
// Copies the verified payload (exactly `size` bytes) into dst and returns the
// saved step in *step; dst is untouched on any error.
Status ReadCheckpoint(const std::string& path, uint64_t plan_hash, uint64_t size, uint8_t* dst,
                      uint64_t* step);

}  // namespace seeml_hip
