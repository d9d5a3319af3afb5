#pragma once
#include <raft/core/mdspan.hpp>
