// Opaque handles of the oracle's C entry points (model, session, scheduler), shared by the
// translation units that expose them — TEST INFRASTRUCTURE ONLY (see oracle.h).
#pragma once

#include <memory>
#include <optional>

#include "oracle_runtime.h"

struct OrcModel {
  std::shared_ptr<orc::Model> model;
};

struct OrcSession {
  std::unique_ptr<orc::Session> session;
};

struct OrcScheduler {
  std::unique_ptr<orc::ReferenceScheduler> sched;
  std::optional<orc::SchedulerReport> last;
  std::unique_ptr<orc::GlobalPagePacker> packer;
  orc::PackedTick packed;
};
