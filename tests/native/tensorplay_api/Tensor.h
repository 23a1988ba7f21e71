#pragma once
#include "api.h"
