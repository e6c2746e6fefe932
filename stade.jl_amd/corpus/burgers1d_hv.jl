function initstacks_burgers1d_b(n, nsteps)
    branch_stack = Vector{Int64}(undef, max(0, div(nsteps - 1, 1) + 1))
    u_stack = Vector{Float64}(undef, max(0, div(nsteps - 1, 1) + 1) * max(0, div(n - 1, 1) + 1))
    return (branch_stack, u_stack)
end

function burgers1d_hv(loss, lossb, u, ub, un, unb, nu, nub, dt, dtb, dx, dxb, tend, tendb, n, nsteps, lossd, lossbd, ud, ubd, und, unbd, nud, nubd, dtd, dtbd, dxd, dxbd, tendd, tendbd, branch_stack, u_stack)
    u_stack_d = Vector{Float64}(undef, length(u_stack))
    cadvb = 0.0
    cadvbd = 0.0
    cdifb = 0.0
    cdifbd = 0.0
    tcb = 0.0
    tcbd = 0.0
    ucb = 0.0
    ucbd = 0.0
    cadvd = (0.5 * dtd) / dx + -((0.5 * dt) / dx ^ 2) * dxd
    cadv = 0.5 * dt / dx
    __hcse_0 = dx * dx
    cdifd = (dt * nud + nu * dtd) / __hcse_0 + -((nu * dt) / __hcse_0 ^ 2) * (dx * dxd + dx * dxd)
    cdif = nu * dt / __hcse_0
    tcd = 0.0
    tc = 0.0
    for i_t = 1:nsteps
        if tc < tend
            __idx_branch_stack_0 = (i_t - 1) + 1
            branch_stack[__idx_branch_stack_0] = 1
            for i_x = 1:n
                im = mod(i_x - 2, n) + 1
                ip = mod(i_x, n) + 1
                ucd = ud[i_x]
                uc = u[i_x]
                __hcse_1 = u[ip] - u[im]
                __hcse_2 = u[ip] - 2.0 * uc + u[im]
                und[i_x] = (ucd + -((uc * __hcse_1) * cadvd + (cadv * __hcse_1) * ucd + (cadv * uc) * (ud[ip] + -(ud[im])))) + (__hcse_2 * cdifd + cdif * ((ud[ip] + -(2.0 * ucd)) + ud[im]))
                un[i_x] = uc - cadv * uc * __hcse_1 + cdif * __hcse_2
            end
            for i_x2 = 1:n
                __idx_u_stack_1 = ((i_x2 - 1) + (i_t - 1) * (div(n - 1, 1) + 1)) + 1
                u_stack_d[__idx_u_stack_1] = ud[i_x2]
                u_stack[__idx_u_stack_1] = u[i_x2]
                ud[i_x2] = und[i_x2]
                u[i_x2] = un[i_x2]
            end
            tcd = tcd + dtd
            tc = tc + dt
        else
            __idx_branch_stack_0 = (i_t - 1) + 1
            branch_stack[__idx_branch_stack_0] = 0
        end
    end
    for i_k = 1:n
        __hcse_3 = u[i_k]
        lossd[1] = lossd[1] + (2__hcse_3) * ud[i_k]
        loss[1] = loss[1] + __hcse_3 ^ 2
    end
    for i_k = n:-1:1
        __hcse_4 = lossb[1]
        __hcse_5 = 2 * u[i_k]
        ubd[i_k] = ubd[i_k] + (__hcse_4 * (2 * ud[i_k]) + __hcse_5 * lossbd[1])
        ub[i_k] = ub[i_k] + __hcse_5 * __hcse_4
    end
    for i_t = nsteps:-1:1
        __idx_branch_stack_0 = (i_t - 1) + 1
        __branch = branch_stack[__idx_branch_stack_0]
        if __branch == 1
            dtbd = dtbd + tcbd
            dtb = dtb + tcb
            for i_x2 = n:-1:1
                __idx_u_stack_1 = ((i_x2 - 1) + (i_t - 1) * (div(n - 1, 1) + 1)) + 1
                ud[i_x2] = u_stack_d[__idx_u_stack_1]
                u[i_x2] = u_stack[__idx_u_stack_1]
                __oldb_1d = ubd[i_x2]
                __oldb_1 = ub[i_x2]
                ubd[i_x2] = 0.0
                ub[i_x2] = 0.0
                unbd[i_x2] = unbd[i_x2] + __oldb_1d
                unb[i_x2] = unb[i_x2] + __oldb_1
            end
            for i_x = n:-1:1
                im = mod(i_x - 2, n) + 1
                ip = mod(i_x, n) + 1
                ucd = ud[i_x]
                uc = u[i_x]
                __oldb_2d = unbd[i_x]
                __oldb_2 = unb[i_x]
                unbd[i_x] = 0.0
                unb[i_x] = 0.0
                __cse_3d = ud[ip] + -(ud[im])
                __cse_3 = u[ip] - u[im]
                __cse_4d = -__oldb_2d
                __cse_4 = -__oldb_2
                ucbd = ucbd + __oldb_2d
                ucb = ucb + __oldb_2
                __hcse_6 = uc * __cse_3
                cadvbd = cadvbd + (__cse_4 * (__cse_3 * ucd + uc * __cse_3d) + __hcse_6 * __cse_4d)
                cadvb = cadvb + __hcse_6 * __cse_4
                __hcse_7 = cadv * __cse_3
                ucbd = ucbd + (__cse_4 * (__cse_3 * cadvd + cadv * __cse_3d) + __hcse_7 * __cse_4d)
                ucb = ucb + __hcse_7 * __cse_4
                __cse_5d = uc * cadvd + cadv * ucd
                __cse_5 = cadv * uc
                __hcse_8 = __cse_4 * __cse_5d + __cse_5 * __cse_4d
                ubd[ip] = ubd[ip] + __hcse_8
                ub[ip] = ub[ip] + __cse_5 * __cse_4
                ubd[im] = ubd[im] + -__hcse_8
                ub[im] = ub[im] + -(__cse_5 * __cse_4)
                __hcse_9d = (ud[ip] + -(2.0 * ucd)) + ud[im]
                __hcse_9 = u[ip] - 2.0 * uc + u[im]
                cdifbd = cdifbd + (__oldb_2 * __hcse_9d + __hcse_9 * __oldb_2d)
                cdifb = cdifb + __hcse_9 * __oldb_2
                __cse_6d = __oldb_2 * cdifd + cdif * __oldb_2d
                __cse_6 = cdif * __oldb_2
                ubd[ip] = ubd[ip] + __cse_6d
                ub[ip] = ub[ip] + __cse_6
                ucbd = ucbd + 2.0 * -__cse_6d
                ucb = ucb + 2.0 * -__cse_6
                ubd[im] = ubd[im] + __cse_6d
                ub[im] = ub[im] + __cse_6
                __oldb_7d = ucbd
                __oldb_7 = ucb
                ucbd = 0.0
                ucb = 0.0
                ubd[i_x] = ubd[i_x] + __oldb_7d
                ub[i_x] = ub[i_x] + __oldb_7
            end
        end
    end
    __oldb_8d = cdifbd
    __oldb_8 = cdifb
    cdifbd = 0.0
    cdifb = 0.0
    __cse_9d = dx * dxd + dx * dxd
    __cse_9 = dx * dx
    __hcse_10d = dtd / __cse_9 + -(dt / __cse_9 ^ 2) * __cse_9d
    __hcse_10 = dt / __cse_9
    nubd = nubd + (__oldb_8 * __hcse_10d + __hcse_10 * __oldb_8d)
    nub = nub + __hcse_10 * __oldb_8
    __hcse_11d = nud / __cse_9 + -(nu / __cse_9 ^ 2) * __cse_9d
    __hcse_11 = nu / __cse_9
    dtbd = dtbd + (__oldb_8 * __hcse_11d + __hcse_11 * __oldb_8d)
    dtb = dtb + __hcse_11 * __oldb_8
    __hcse_12d = dt * nud + nu * dtd
    __hcse_12 = nu * dt
    __hcse_13d = (2__cse_9) * __cse_9d
    __hcse_13 = __cse_9 ^ 2
    __cse_10d = -(__hcse_12 / __hcse_13) * __oldb_8d + -(__hcse_12d / __hcse_13 + -(__hcse_12 / __hcse_13 ^ 2) * __hcse_13d) * __oldb_8
    __cse_10 = -(__hcse_12 / __hcse_13) * __oldb_8
    dxbd = dxbd + (__cse_10 * dxd + dx * __cse_10d)
    dxb = dxb + dx * __cse_10
    dxbd = dxbd + (__cse_10 * dxd + dx * __cse_10d)
    dxb = dxb + dx * __cse_10
    __oldb_11d = cadvbd
    __oldb_11 = cadvb
    cadvbd = 0.0
    cadvb = 0.0
    __hcse_14d = -(0.5 / dx ^ 2) * dxd
    __hcse_14 = 0.5 / dx
    dtbd = dtbd + (__oldb_11 * __hcse_14d + __hcse_14 * __oldb_11d)
    dtb = dtb + __hcse_14 * __oldb_11
    __hcse_15d = -((0.5 * dtd) / dx ^ 2 + -((0.5 * dt) / (dx ^ 2) ^ 2) * ((2dx) * dxd))
    __hcse_15 = -((0.5 * dt) / dx ^ 2)
    dxbd = dxbd + (__oldb_11 * __hcse_15d + __hcse_15 * __oldb_11d)
    dxb = dxb + __hcse_15 * __oldb_11
    return (nub, nubd, dtb, dtbd, dxb, dxbd, tendb, tendbd)
end

function burgers1d(loss, u, un, nu, dt, dx, tend, n, nsteps)
    cadv = 0.5 * dt / dx
    cdif = nu * dt / (dx * dx)
    tc = 0.0
    for i_t = 1:nsteps
        if tc < tend
            for i_x = 1:n
                im = mod(i_x - 2, n) + 1
                ip = mod(i_x, n) + 1
                uc = u[i_x]
                un[i_x] = uc - cadv * uc * (u[ip] - u[im]) + cdif * (u[ip] - 2.0 * uc + u[im])
            end
            for i_x2 = 1:n
                u[i_x2] = un[i_x2]
            end
            tc = tc + dt
        end
    end
    for i_k = 1:n
        loss[1] = loss[1] + u[i_k] ^ 2
    end
    return nothing
end
